// Shared helpers for the gfx950 Sol-Attn kernels: error reporting, bf16
// conversion, MFMA operand types and small wave-level utilities.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/solattn.h"

namespace solattn {

// Records a message for solattn_last_error() and returns code (capi.hip).
int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

// Checks the launch that was just issued; returns 0 or SOLATTN_ELAUNCH.
int check_launch(const char* what);

#define SOLATTN_REQUIRE(cond, code, ...)                \
  do {                                                  \
    if (!(cond)) return ::solattn::set_error((code), __VA_ARGS__); \
  } while (0)

typedef __attribute__((__vector_size__(8 * sizeof(__bf16)))) __bf16 bf16x8;
typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4;
typedef __attribute__((__vector_size__(2 * sizeof(__bf16)))) __bf16 bf16x2;
typedef __attribute__((__vector_size__(16 * sizeof(float)))) float f32x16;
typedef __attribute__((__vector_size__(4 * sizeof(float)))) float f32x4;
typedef __attribute__((__vector_size__(4 * sizeof(int)))) int i32x4;
typedef __attribute__((__vector_size__(16 * sizeof(int)))) int i32x16;
typedef __attribute__((__vector_size__(2 * sizeof(int)))) int i32x2;

__device__ __forceinline__ float bf2f(uint16_t h) {
  return __uint_as_float(static_cast<uint32_t>(h) << 16);
}

// Round-to-nearest-even fp32 -> bf16 bits; same rule as the CPU oracle.
__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return static_cast<uint16_t>((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return static_cast<uint16_t>(u >> 16);
}

__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  return static_cast<uint32_t>(f2bf(lo)) | (static_cast<uint32_t>(f2bf(hi)) << 16);
}

// Two fp32 -> a packed bf16 pair (lo, hi) in one v_cvt_pk_bf16_f32: round to
// nearest even, the bits of f2bf for every non-NaN input (denormals included:
// f32 denormals are not flushed in this build).
__device__ __forceinline__ uint32_t cvt_pk_bf16(float lo, float hi) {
  typedef __attribute__((ext_vector_type(2))) float f2;
  typedef __attribute__((ext_vector_type(2))) __bf16 h2;
  const f2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, h2));
}

__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// Raw buffer access: base is wave-uniform (a scalar resource), off a per-lane
// byte offset (one VGPR instead of a 64-bit address per load). The hardware
// range check returns zeros for a 16-byte load whose end passes nbytes (and
// drops such a store); callers keep each 16-byte access wholly inside or
// wholly past nbytes. Word 3 0x00020000: 32-bit data format, no swizzle.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t nbytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, static_cast<int>(nbytes),
                                           0x00020000);
}
__device__ __forceinline__ uint4 buffer_load16(const void* base, uint32_t nbytes, uint32_t off) {
  const auto v = __builtin_amdgcn_raw_buffer_load_b128(buffer_rsrc(base, nbytes), off, 0, 0);
  return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ uint32_t buffer_load4(const void* base, uint32_t nbytes, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b32(buffer_rsrc(base, nbytes), off, 0, 0);
}
__device__ __forceinline__ uint16_t buffer_load2(const void* base, uint32_t nbytes, uint32_t off) {
  return __builtin_amdgcn_raw_buffer_load_b16(buffer_rsrc(base, nbytes), off, 0, 0);
}
__device__ __forceinline__ void buffer_store2(void* base, uint32_t nbytes, uint32_t off, uint16_t x) {
  __builtin_amdgcn_raw_buffer_store_b16(x, buffer_rsrc(base, nbytes), off, 0, 0);
}
__device__ __forceinline__ void buffer_store16(void* base, uint32_t nbytes, uint32_t off,
                                               const uint4& x) {
  typedef __attribute__((__vector_size__(4 * sizeof(uint32_t)))) uint32_t u32x4;
  const u32x4 v = {x.x, x.y, x.z, x.w};
  __builtin_amdgcn_raw_buffer_store_b128(v, buffer_rsrc(base, nbytes), off, 0, 0);
}

// Bytes of a row-strided buffer that rows [r, n) span when the last row ends
// `tail` bytes after its start (row pitch `pitch` bytes), capped at `cap`: the
// nbytes of buffer_load16 for a base at row r; 0 when r >= n.
__device__ __forceinline__ uint32_t rows_nbytes(int64_t r, int64_t n, int64_t pitch, int64_t tail,
                                                int64_t cap) {
  if (r >= n) return 0u;
  const int64_t bytes = (n - 1 - r) * pitch + tail;
  return static_cast<uint32_t>(bytes < cap ? bytes : cap);
}

constexpr float kLog2e = 1.4426950408889634f;

inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// The pooling pass (prep.hip) with, when qi != null, the per-token INT8 of q
// (codes qi [B, TP, H, 128], scales qs [B, TP, H]) in the same read;
// pool_checked validates the arguments as solattn_pool does.
int pool_checked(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t* k,
                 int64_t sk_b, int64_t sk_t, int64_t sk_h, const uint16_t* v, int64_t sv_b,
                 int64_t sv_t, int64_t sv_h, int64_t B, int64_t T, int64_t H, int64_t D,
                 int64_t block, uint16_t* kc, uint16_t* vc, int64_t npad, float* qbar,
                 float* vamax_part, int8_t* qi, float* qs, int64_t TP, hipStream_t s);
int launch_pool(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t* k,
                int64_t sk_b, int64_t sk_t, int64_t sk_h, const uint16_t* v, int64_t sv_b,
                int64_t sv_t, int64_t sv_h, int64_t B, int64_t T, int64_t H, int64_t block,
                uint16_t* kc, uint16_t* vc, int64_t npad, float* qbar, float* vamax_part,
                int8_t* qi, float* qs, int64_t TP, hipStream_t s);

// The INT8 preparation with one read of q, k and v (prep.hip): pooled keys,
// centred kc, moments, V scale, Q/K/V codes; as solattn_prep_int8, whose
// SOLATTN_EUNSUPPORTED means: use pool -> moments -> quant instead.
int64_t single_read_sync_words(int64_t B, int64_t H);
int prep_int8_single_read(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                          const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                          const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                          int64_t T, int64_t H, int64_t D, int64_t block, uint16_t* kc,
                          uint16_t* vc, int64_t npad, float* qbar, float* kc_mean, float* kc_var,
                          float* vamax_part, float* vscale, int8_t* qi, float* qs, int8_t* ki,
                          float* ks, int ks_head_major, int8_t* vi, int64_t TP, uint32_t* sync,
                          int64_t sync_bytes, hipStream_t stream);

// Copies BTHD rows of din bf16 channels into rows of dout channels, zero
// filled (din < dout), or the first dout channels back out (din > dout)
// (reorder.hip).
int pad_heads(const uint16_t* src, int64_t s_b, int64_t s_t, int64_t s_h, uint16_t* dst,
              int64_t d_b, int64_t d_t, int64_t d_h, int64_t B, int64_t T, int64_t H, int64_t din,
              int64_t dout, hipStream_t stream);

// Per-token INT8 of q (skipped when q is null) and of k smoothed by k_mean,
// and (vscale != null) per-channel INT8 of v, in one launch (quant.hip); same
// codes and scales as solattn_quant_rows / solattn_quant_v (qk_block: q and k
// as solattn_quant_rows_blocked); ks_head_major: k's scales laid out [B, H, TP]
// instead of [B, TP, H].
int quant_qkv(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t* k,
              int64_t sk_b, int64_t sk_t, int64_t sk_h, const uint16_t* v, int64_t sv_b,
              int64_t sv_t, int64_t sv_h, int64_t B, int64_t T, int64_t H, int64_t D,
              const float* k_mean, const float* vscale, int8_t* qi, float* qs, int8_t* ki,
              float* ks, int8_t* vi, int64_t TP, hipStream_t stream, int qk_block = 0,
              int ks_head_major = 0);

// solattn_fwd_int8 without clearing the error slot; uniform_ks: every 64-key
// tile of K shares one scale (K quantised per 128-token block), so the
// kernels multiply it once per tile instead of once per score; ks_head_major:
// ks laid out [B, H, TP] (a tile's 64 scales contiguous) instead of [B, TP, H].
int fwd_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const int8_t* qi,
             const float* qs, const int8_t* ki, const float* ks, const int8_t* vi,
             const float* vscale, const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
             int64_t TP, const uint16_t* kc, const uint16_t* vc, int64_t npad,
             const int32_t* counts, const uint32_t* mask, int64_t B,
             int64_t T, int64_t H, int64_t D, int64_t block, float scale, int int8_pv,
             uint16_t* o, int64_t so_b, int64_t so_t, int64_t so_h, solattn_stream_t stream,
             bool uniform_ks, bool ks_head_major = false);

}  // namespace solattn
