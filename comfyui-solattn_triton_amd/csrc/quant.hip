// Per-token and per-channel INT8 quantisation for the Sol-Attn INT8 path.
//
// Built with -ffp-contract=off; divisions are IEEE (HIP's default correctly
// rounded fp32 divide), so codes and scales match the CPU oracle bit for bit.
// One row (token, head) of 128 channels is held by 16 lanes x 8 channels; the
// row's |max| is reduced with DPP lane moves inside the 16-lane group.
#include "common.hpp"
#include "quant_common.hpp"

namespace solattn {

constexpr int kQD = 128;
constexpr int kQuantThreads = 256;
constexpr int kRowsPerWG = kQuantThreads / 16;

// One launch quantises up to three BTHD tensors (blockIdx.z picks the
// tensor): per token with an optional smoothing mean (Q, K;
// /root/reference/_fused_quant.py:8-42 and the Q half of
// /root/reference/_fused_prep.py:42-48, whose clamp-then-round gives the same
// codes) or per channel against vscale (V; /root/reference/_fused_quant.py:61-88).
// A workgroup owns kQuantTok tokens of one (batch, head): its 16 lane groups
// take tokens t0 + g, t0 + g + 16, ... and each lane 8 channels, so the mean
// or channel scales sit in registers for the whole workgroup and every lane
// has kQuantR 16-byte row loads in flight before any arithmetic.
//
// Codes and scales follow quant_common.hpp.
constexpr int kQuantR = 8;                       // tokens per lane group
constexpr int kQuantTok = kQuantR * kRowsPerWG;  // tokens per workgroup
static_assert(kQuantTok == SOLATTN_QUANT_BLOCK, "a workgroup quantises one scale block");

struct QuantTensor {
  const uint16_t* x;
  int64_t sb, st, sh;     // element strides of x
  const float* mean;      // [B, H, D] smoothing mean, or null
  const float* vscale;    // [B, H, D] per-channel scale (V rule), or null
  int8_t* xi;             // [B, TP, H, D]
  float* xs;              // per-token scales (not written by the V rule)
  int block_scale;        // per-token rule with one scale per kQuantTok-token block
  // element strides of xs within a batch's TP*H scales: token-major [B, TP, H]
  // (xs_st = H, xs_sh = 1, as the reference's) or head-major [B, H, TP]
  // (xs_st = 1, xs_sh = TP, the INT8 call's own K scales)
  int64_t xs_st, xs_sh;
};

struct QuantArgs {
  QuantTensor t[3];
  uint32_t T, H;
  int64_t TP;
};

// The eight bf16 of a 16-byte load minus the smoothing mean (0 without one).
__device__ __forceinline__ void smoothed(const uint4& raw, const float (&m)[8], float (&y)[8]) {
  const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    y[2 * e] = lo_bf16(w[e]) - m[2 * e];
    y[2 * e + 1] = hi_bf16(w[e]) - m[2 * e + 1];
  }
}

// PER_CHANNEL: V against vscale[d]; otherwise per token (or per block with
// block_scale), smoothed by mean when the tensor has one.
template <bool PER_CHANNEL>
__device__ __forceinline__ void quant_rows_of(const QuantTensor& A, uint32_t T, uint32_t H,
                                              int64_t TP) {
  const uint32_t bh = blockIdx.x, b = bh / H, h = bh % H;
  const int c8 = (threadIdx.x & 15) * 8;
  const uint32_t t0 = blockIdx.y * kQuantTok + (threadIdx.x >> 4);
  const uint16_t* xb = A.x + b * A.sb + h * A.sh + c8;

  uint4 raw[kQuantR];
#pragma unroll
  for (int r = 0; r < kQuantR; ++r) {  // tokens past T re-read token T-1; nothing is stored
    const uint32_t t = min(t0 + r * kRowsPerWG, T - 1);
    raw[r] = *reinterpret_cast<const uint4*>(xb + static_cast<int64_t>(t) * A.st);
  }
  const int64_t chan = static_cast<int64_t>(bh) * kQD + c8;
  float m[8], sv[8], rs[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    m[e] = (!PER_CHANNEL && A.mean) ? A.mean[chan + e] : 0.f;
    sv[e] = PER_CHANNEL ? A.vscale[chan + e] : 1.f;
    rs[e] = PER_CHANNEL ? __builtin_amdgcn_rcpf(sv[e]) : 1.f;
  }

  // Per-block rule: the |max| of the workgroup's tokens (one kQuantTok-token
  // block of one head; tokens past T repeat token T-1 of the same block), over
  // the 16 lanes of a row by DPP and over the 16 rows through LDS.
  float block_ss = 0.f;
  float block_rr[8], block_sv[8];
  if (!PER_CHANNEL && A.block_scale) {
    __shared__ uint32_t srow_max[kRowsPerWG];
    uint32_t mb = 0;
#pragma unroll
    for (int r = 0; r < kQuantR; ++r) {
      float y[8];
      smoothed(raw[r], m, y);
#pragma unroll
      for (int e = 0; e < 8; ++e) mb = max(mb, __float_as_uint(y[e]) & 0x7fffffffu);
    }
    mb = group16_max_bits(mb);
    if ((threadIdx.x & 15) == 0) srow_max[threadIdx.x >> 4] = mb;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < kRowsPerWG; ++i) mb = max(mb, srow_max[i]);
    const float sc = div127(__uint_as_float(mb));
    block_ss = sc > 1e-8f ? sc : 1e-8f;
    const float rr = __builtin_amdgcn_rcpf(block_ss);
#pragma unroll
    for (int e = 0; e < 8; ++e) block_rr[e] = rr, block_sv[e] = block_ss;
  }

#pragma unroll
  for (int r = 0; r < kQuantR; ++r) {
    const uint32_t t = t0 + r * kRowsPerWG;
    float y[8];
    smoothed(raw[r], m, y);
    float ss = 1.f;
    uint2 o;
    if (!PER_CHANNEL && block_ss > 0.f) {  // the block's scale
      ss = block_ss;
      o = codes8(y, block_rr, block_sv);
    } else if (!PER_CHANNEL) {
      ss = quant_token_row(y, o);
    } else {
      o = codes8(y, rs, sv);
    }
    if (t < T) {
      const int64_t row = (static_cast<int64_t>(b) * TP + t) * H + h;
      *reinterpret_cast<uint2*>(A.xi + row * kQD + c8) = o;
      if (!PER_CHANNEL && (threadIdx.x & 15) == 0)
        A.xs[static_cast<int64_t>(b) * TP * H + t * A.xs_st + h * A.xs_sh] = ss;
    }
  }
}

__global__ void __launch_bounds__(kQuantThreads)
quant3_kernel(const QuantArgs args) {
  // Heads vary fastest over the grid, so the workgroups in flight read
  // neighbouring tokens of every head: contiguous memory for a BTHD tensor.
  const QuantTensor& A = args.t[blockIdx.z];
  if (A.vscale != nullptr)
    quant_rows_of<true>(A, args.T, args.H, args.TP);
  else
    quant_rows_of<false>(A, args.T, args.H, args.TP);
}

int check_quant_tensor(const QuantTensor& q, int64_t B, int64_t T, int64_t H, int64_t TP,
                       const char* what) {
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && TP >= T, SOLATTN_EINVAL, "%s: bad sizes", what);
  SOLATTN_REQUIRE(B * H < (1ll << 31) && cdiv(T, kQuantTok) <= 65535, SOLATTN_EUNSUPPORTED,
                  "%s: too many rows", what);
  SOLATTN_REQUIRE(q.x && q.xi && (q.vscale || q.xs), SOLATTN_EINVAL, "%s: null pointer", what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(q.x) % 16 == 0 && q.sb % 8 == 0 && q.st % 8 == 0 &&
                      q.sh % 8 == 0 && reinterpret_cast<uintptr_t>(q.xi) % 8 == 0,
                  SOLATTN_EINVAL, "%s: unaligned input or strides", what);
  return 0;
}

// Quantises n (1..3) tensors of the same B, T, H in one launch.
int launch_quant3(const QuantTensor* ts, int n, int64_t B, int64_t T, int64_t H, int64_t D,
                  int64_t TP, hipStream_t stream, const char* what) {
  SOLATTN_REQUIRE(D == kQD, SOLATTN_EUNSUPPORTED, "%s: head_dim %lld != 128", what, (long long)D);
  SOLATTN_REQUIRE(n >= 1 && n <= 3, SOLATTN_EINVAL, "%s: %d tensors", what, n);
  QuantArgs args{};
  for (int i = 0; i < n; ++i) {
    if (int rc = check_quant_tensor(ts[i], B, T, H, TP, what)) return rc;
    args.t[i] = ts[i];
  }
  args.T = static_cast<uint32_t>(T);
  args.H = static_cast<uint32_t>(H);
  args.TP = TP;
  dim3 grid(static_cast<uint32_t>(B * H), static_cast<uint32_t>(cdiv(T, kQuantTok)),
            static_cast<uint32_t>(n));
  hipLaunchKernelGGL(quant3_kernel, grid, dim3(kQuantThreads), 0, stream, args);
  return check_launch(what);
}

int launch_quant(const uint16_t* x, int64_t sx_b, int64_t sx_t, int64_t sx_h, int64_t B,
                 int64_t T, int64_t H, int64_t D, const float* mean, const float* vscale,
                 int8_t* xi, float* xs, int64_t TP, hipStream_t stream, const char* what,
                 int block_scale = 0) {
  const QuantTensor t{x, sx_b, sx_t, sx_h, mean, vscale, xi, xs, block_scale, H, 1};
  return launch_quant3(&t, 1, B, T, H, D, TP, stream, what);
}

int quant_qkv(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t* k,
              int64_t sk_b, int64_t sk_t, int64_t sk_h, const uint16_t* v, int64_t sv_b,
              int64_t sv_t, int64_t sv_h, int64_t B, int64_t T, int64_t H, int64_t D,
              const float* k_mean, const float* vscale, int8_t* qi, float* qs, int8_t* ki,
              float* ks, int8_t* vi, int64_t TP, hipStream_t stream, int qk_block,
              int ks_head_major) {
  QuantTensor ts[3];
  int n = 0;
  if (q) ts[n++] = {q, sq_b, sq_t, sq_h, nullptr, nullptr, qi, qs, qk_block, H, 1};
  ts[n++] = {k, sk_b, sk_t, sk_h, k_mean, nullptr, ki, ks, qk_block, ks_head_major ? 1 : H,
             ks_head_major ? TP : 1};
  if (vscale) ts[n++] = {v, sv_b, sv_t, sv_h, nullptr, vscale, vi, nullptr, 0, H, 1};
  return launch_quant3(ts, n, B, T, H, D, TP, stream, "quant_qkv");
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

extern "C" int solattn_quant_rows_blocked(const uint16_t* x, int64_t sx_b, int64_t sx_t,
                                          int64_t sx_h, int64_t B, int64_t T, int64_t H,
                                          int64_t D, const float* mean, int8_t* xi, float* xs,
                                          int64_t TP, solattn_stream_t stream) {
  clear_error();
  return launch_quant(x, sx_b, sx_t, sx_h, B, T, H, D, mean, nullptr, xi, xs, TP,
                      reinterpret_cast<hipStream_t>(stream), "quant_rows_blocked", 1);
}

extern "C" int solattn_quant_v(const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                               int64_t B, int64_t T, int64_t H, int64_t D, const float* vscale,
                               int8_t* vi, int64_t TP, solattn_stream_t stream) {
  clear_error();
  SOLATTN_REQUIRE(vscale != nullptr, SOLATTN_EINVAL, "quant_v: null vscale");
  return launch_quant(v, sv_b, sv_t, sv_h, B, T, H, D, nullptr, vscale, vi, nullptr, TP,
                      reinterpret_cast<hipStream_t>(stream), "quant_v");
}
