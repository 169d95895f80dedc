// Per-token and per-channel INT8 quantisation for the Sol-Attn INT8 path.
//
// Built with -ffp-contract=off; divisions are IEEE (HIP's default correctly
// rounded fp32 divide), so codes and scales match the CPU oracle bit for bit.
// One row (token, head) of 128 channels is held by 16 lanes x 8 channels; the
// row's |max| is reduced with 4 xor shuffles inside the 16-lane group.
#include "common.hpp"

namespace solattn {

constexpr int kQD = 128;
constexpr int kQuantThreads = 256;
constexpr int kRowsPerWG = kQuantThreads / 16;

// trunc(val + copysign(0.5, val)) clamped to [-127, 127]: the reference's
// val >= 0 ? trunc(val + 0.5) : trunc(val - 0.5) as an integer for every
// float (at val = -0 both give 0).
__device__ __forceinline__ int8_t round_half_away_clamp(float val) {
  float r = truncf(val + copysignf(0.5f, val));
  r = fminf(fmaxf(r, -127.f), 127.f);
  return static_cast<int8_t>(static_cast<int>(r));
}

__device__ __forceinline__ uint32_t pack_i8x4(int8_t a, int8_t b, int8_t c, int8_t d) {
  return static_cast<uint32_t>(static_cast<uint8_t>(a)) |
         (static_cast<uint32_t>(static_cast<uint8_t>(b)) << 8) |
         (static_cast<uint32_t>(static_cast<uint8_t>(c)) << 16) |
         (static_cast<uint32_t>(static_cast<uint8_t>(d)) << 24);
}

// /root/reference/_fused_quant.py:8-42 (per token, optional smoothing mean)
// and /root/reference/_fused_prep.py:42-48 (Q; clamp-then-round gives the
// same codes). vscale != nullptr switches to the per-channel V rule,
// /root/reference/_fused_quant.py:61-88. Each 16-lane group handles kRowsPerGroup
// rows, kQuantThreads / 16 groups apart, with every row's load issued before
// any arithmetic (more bytes in flight per lane).
constexpr int kRowsPerGroup = 4;
constexpr int kRowsPerChunk = kRowsPerGroup * kRowsPerWG;  // rows of one workgroup pass

// The rows of one chunk a lane group owns: 16-byte loads and their (b, t, h).
struct QuantRows {
  uint32_t rw[kRowsPerGroup], hh[kRowsPerGroup], tt[kRowsPerGroup], bb[kRowsPerGroup];
  uint4 raw[kRowsPerGroup];
};

__device__ __forceinline__ void quant_load(QuantRows& R, uint32_t chunk, const uint16_t* __restrict__ x,
                                           int64_t sx_b, int64_t sx_t, int64_t sx_h, uint32_t T,
                                           uint32_t H, uint32_t rows, int c8) {
  // (b, t, h) of the first row by division, of the others by stepping
  // kRowsPerWG rows forward (rows are ordered b, t, h with h fastest).
  const uint32_t row0 = chunk * kRowsPerChunk + (threadIdx.x >> 4);
  uint32_t hc = row0 % H, bt = row0 / H;
  uint32_t tc = bt % T, bc = bt / T;
#pragma unroll
  for (int k = 0; k < kRowsPerGroup; ++k) {
    R.rw[k] = row0 + k * kRowsPerWG;
    const bool in = R.rw[k] < rows;
    // rows past the end re-read the last row (loads stay in bounds; nothing is stored)
    R.hh[k] = in ? hc : H - 1;
    R.tt[k] = in ? tc : T - 1;
    R.bb[k] = in ? bc : (rows / H) / T - 1;
    R.raw[k] = *reinterpret_cast<const uint4*>(x + R.bb[k] * sx_b +
                                               static_cast<int64_t>(R.tt[k]) * sx_t + R.hh[k] * sx_h + c8);
    hc += kRowsPerWG;
    while (hc >= H) {  // at most kRowsPerWG / H + 1 steps
      hc -= H;
      if (++tc == T) {
        tc = 0;
        ++bc;
      }
    }
  }
}

// One chunk of kRowsPerChunk rows per workgroup.
__global__ void __launch_bounds__(kQuantThreads)
quant_kernel(const uint16_t* __restrict__ x, int64_t sx_b, int64_t sx_t, int64_t sx_h,
             uint32_t T, uint32_t H, uint32_t rows, const float* __restrict__ mean,
             const float* __restrict__ vscale, int8_t* __restrict__ xi, float* __restrict__ xs,
             int64_t TP) {
  const int c8 = (threadIdx.x & 15) * 8;
  {
    QuantRows cur;
    quant_load(cur, blockIdx.x, x, sx_b, sx_t, sx_h, T, H, rows, c8);
    const uint32_t* rw = cur.rw;
    const uint32_t* hh = cur.hh;
    const uint32_t* tt = cur.tt;
    const uint32_t* bb = cur.bb;
    const uint4* raw = cur.raw;
#pragma unroll
    for (int k = 0; k < kRowsPerGroup; ++k) {
      const uint32_t b = bb[k], t = tt[k], h = hh[k];
      const uint32_t w[4] = {raw[k].x, raw[k].y, raw[k].z, raw[k].w};
      float y[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        y[2 * e] = lo_bf16(w[e]);
        y[2 * e + 1] = hi_bf16(w[e]);
      }
      const int64_t bh = static_cast<int64_t>(b) * H + h;
      int8_t code[8];
      if (vscale) {
        const float4* sp = reinterpret_cast<const float4*>(vscale + bh * kQD + c8);
        const float4 s0 = sp[0], s1 = sp[1];
        const float sv[8] = {s0.x, s0.y, s0.z, s0.w, s1.x, s1.y, s1.z, s1.w};
#pragma unroll
        for (int e = 0; e < 8; ++e) code[e] = round_half_away_clamp(y[e] / sv[e]);
      } else {
        if (mean) {
          const float4* mp = reinterpret_cast<const float4*>(mean + bh * kQD + c8);
          const float4 m0 = mp[0], m1 = mp[1];
          const float m[8] = {m0.x, m0.y, m0.z, m0.w, m1.x, m1.y, m1.z, m1.w};
#pragma unroll
          for (int e = 0; e < 8; ++e) y[e] = y[e] - m[e];
        }
        float amax = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(y[e]));
#pragma unroll
        for (int sh = 1; sh < 16; sh <<= 1) amax = fmaxf(amax, __shfl_xor(amax, sh));
        const float sc = amax / 127.0f;
        const float ss = sc > 1e-8f ? sc : 1e-8f;
        // y * fl(1/ss) is within 2.3e-5 of the IEEE quotient fl(y/ss) (|y/ss| <=
        // 127.5; fl(1/ss), the product and the quotient each round by <= 2^-24
        // relative), so the codes agree unless that quotient lies within 3e-5 of
        // k + 0.5; lanes with such a value redo their 8 channels by IEEE division.
        const float r = 1.0f / ss;
        bool near = false;
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float q1 = y[e] * r;
          const float a = fabsf(q1);
          near |= fabsf((a - truncf(a)) - 0.5f) <= 3e-5f;
          code[e] = round_half_away_clamp(q1);
        }
        if (near) {
          asm volatile("");  // keeps the divisions on this rare path
#pragma unroll
          for (int e = 0; e < 8; ++e) code[e] = round_half_away_clamp(y[e] / ss);
        }
        if ((threadIdx.x & 15) == 0 && rw[k] < rows) xs[(static_cast<int64_t>(b) * TP + t) * H + h] = ss;
      }
      if (rw[k] < rows) {
        uint2 o;
        o.x = pack_i8x4(code[0], code[1], code[2], code[3]);
        o.y = pack_i8x4(code[4], code[5], code[6], code[7]);
        *reinterpret_cast<uint2*>(xi + ((static_cast<int64_t>(b) * TP + t) * H + h) * kQD + c8) = o;
      }
    }
  }
}

int launch_quant(const uint16_t* x, int64_t sx_b, int64_t sx_t, int64_t sx_h, int64_t B,
                 int64_t T, int64_t H, int64_t D, const float* mean, const float* vscale,
                 int8_t* xi, float* xs, int64_t TP, hipStream_t stream, const char* what) {
  SOLATTN_REQUIRE(D == kQD, SOLATTN_EUNSUPPORTED, "%s: head_dim %lld != 128", what, (long long)D);
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && TP >= T, SOLATTN_EINVAL, "%s: bad sizes", what);
  SOLATTN_REQUIRE(B * T * H < (1ll << 31), SOLATTN_EUNSUPPORTED, "%s: too many rows", what);
  SOLATTN_REQUIRE(x && xi && (vscale || xs), SOLATTN_EINVAL, "%s: null pointer", what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(x) % 16 == 0 && sx_b % 8 == 0 && sx_t % 8 == 0 &&
                      sx_h % 8 == 0 && reinterpret_cast<uintptr_t>(xi) % 8 == 0,
                  SOLATTN_EINVAL, "%s: unaligned input or strides", what);
  const uint32_t rows = static_cast<uint32_t>(B * T * H);
  hipLaunchKernelGGL(quant_kernel, dim3(static_cast<uint32_t>(cdiv(rows, kRowsPerChunk))),
                     dim3(kQuantThreads), 0, stream, x, sx_b, sx_t, sx_h,
                     static_cast<uint32_t>(T), static_cast<uint32_t>(H), rows, mean, vscale, xi,
                     xs, TP);
  return check_launch(what);
}

}  // namespace solattn

using namespace solattn;

extern "C" int solattn_quant_rows(const uint16_t* x, int64_t sx_b, int64_t sx_t, int64_t sx_h,
                                  int64_t B, int64_t T, int64_t H, int64_t D, const float* mean,
                                  int8_t* xi, float* xs, int64_t TP, solattn_stream_t stream) {
  clear_error();
  return launch_quant(x, sx_b, sx_t, sx_h, B, T, H, D, mean, nullptr, xi, xs, TP,
                      reinterpret_cast<hipStream_t>(stream), "quant_rows");
}

extern "C" int solattn_quant_v(const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                               int64_t B, int64_t T, int64_t H, int64_t D, const float* vscale,
                               int8_t* vi, int64_t TP, solattn_stream_t stream) {
  clear_error();
  SOLATTN_REQUIRE(vscale != nullptr, SOLATTN_EINVAL, "quant_v: null vscale");
  return launch_quant(v, sv_b, sv_t, sv_h, B, T, H, D, nullptr, vscale, vi, nullptr, TP,
                      reinterpret_cast<hipStream_t>(stream), "quant_v");
}
