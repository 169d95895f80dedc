// Pooling, moments, thresholds and routing for Sol-Attn on gfx950.
//
// Built with -ffp-contract=off: every fp32 operation below is rounded exactly
// where it is written, so the CPU oracle (oracle/solattn_oracle.c) reproduces
// kc, vc, qbar, thresholds and routing masks bit for bit.
//
//  pool    one pass over q, k, v: a workgroup per 128 rows of one head,
//          sixteen row slots (rows g mod 16), each lane 8 channels in 16-byte
//          loads; HBM-bound; optionally quantises Q on the way (the INT8 path).
//  moments per-head kc mean / variance over blocks (+ INT8 centring, V scale).
//  route   thresholds, scores R[i][j], per-query-block exact masks and counts.
#include <algorithm>

#include "common.hpp"
#include "quant_common.hpp"

namespace solattn {

constexpr int kHeadDim = 128;

// ------------------------------------------------------------------ pool --
// /root/reference/_preprocess.py:23-113 (kc = sum/len, vc = sum, |v| max) and
// the q centroid of :140-149. A workgroup of four waves covers a span of 128
// rows of one head (one block at block 128, two at block 64): wave w, lane
// group u (16 lanes, one DPP row) own slot g = 4w + u, i.e. rows g + 16m
// (m < 8), and each lane 8 channels (16-byte loads). A lane's serial sum over
// the rows of one block is partial p_g of the contract (rows r = g mod 16,
// ascending); the 16 partials meet in LDS and tree16 combines them. All 24
// rows of a lane (Q, K and V) are in flight before any arithmetic.
// With qi != null the pass also quantises each Q row per token
// (/root/reference/_fused_prep.py:42-48, the codes of quant_common.hpp): a
// row's 128 channels are one lane group, so its |max| is a DPP reduction.
constexpr int kSpan = 128;                // rows per workgroup
constexpr int kSlots = 16;                // partials of the pooling contract
constexpr int kSlotRows = kSpan / kSlots; // rows per lane
constexpr int kPoolThreads = 256;

// The eight bf16 of a 16-byte load as floats.
__device__ __forceinline__ void unpack8(const uint4& w, float (&x)[8]) {
  x[0] = lo_bf16(w.x); x[1] = hi_bf16(w.x); x[2] = lo_bf16(w.y); x[3] = hi_bf16(w.y);
  x[4] = lo_bf16(w.z); x[5] = hi_bf16(w.z); x[6] = lo_bf16(w.w); x[7] = hi_bf16(w.w);
}

// The pooling layout of this thread.
struct PoolLane {
  int g;   // slot: rows r0 + g + 16m of the span
  int c8;  // first of the lane's 8 channels
  __device__ __forceinline__ PoolLane()
      : g(4 * static_cast<int>(threadIdx.x >> 6) + static_cast<int>((threadIdx.x >> 4) & 3)),
        c8(static_cast<int>(threadIdx.x & 15) * 8) {}
};

// The lane's kSlotRows rows of one head (xh = x + b*sb + h*sh + c8, row stride
// st) from span row r0; rows past T re-read row T-1 (unconditional loads, so
// all are in flight together; the pooling adds 0.0f for them).
__device__ __forceinline__ void load_span(const uint16_t* xh, int64_t st, int64_t r0, int64_t T,
                                          int g, uint4 (&raw)[kSlotRows]) {
#pragma unroll
  for (int m = 0; m < kSlotRows; ++m)
    raw[m] = *reinterpret_cast<const uint4*>(xh + min(r0 + g + 16 * m, T - 1) * st);
}

// Partial p_g of each block of the span into part[blk][g][c] (LDS, fp32), and
// with AMAX the lane's |max| per block into amx[blk][g][c]; rows past T add
// 0.0f (p + 0.0f == p: a partial that starts at +0.0f never becomes -0.0f).
template <int BLK, bool AMAX>
__device__ __forceinline__ void pool_span(const uint4 (&raw)[kSlotRows], int64_t r0, int64_t T,
                                          const PoolLane& pl, float* part, float* amx) {
  constexpr int NB = kSpan / BLK, RB = kSlotRows / NB;  // blocks per span, lane rows per block
#pragma unroll
  for (int blk = 0; blk < NB; ++blk) {
    float p[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float am[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < RB; ++i) {
      const int m = blk * RB + i;
      const bool valid = r0 + pl.g + 16 * m < T;
      float x[8];
      unpack8(raw[m], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float y = valid ? x[e] : 0.f;
        p[e] = p[e] + y;
        if (AMAX) am[e] = fmaxf(am[e], fabsf(y));
      }
    }
    float4* dst = reinterpret_cast<float4*>(part + ((blk * kSlots + pl.g) * kHeadDim + pl.c8));
    dst[0] = make_float4(p[0], p[1], p[2], p[3]);
    dst[1] = make_float4(p[4], p[5], p[6], p[7]);
    if (AMAX) {
      float4* da = reinterpret_cast<float4*>(amx + ((blk * kSlots + pl.g) * kHeadDim + pl.c8));
      da[0] = make_float4(am[0], am[1], am[2], am[3]);
      da[1] = make_float4(am[4], am[5], am[6], am[7]);
    }
  }
}

// The contract's combination of the 16 partials of one (block, channel),
// p[g * stride]: ((((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7))) + (((p8+p9)+..)..)).
__device__ __forceinline__ float tree16(const float* p, int stride) {
  float a[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) a[i] = p[(2 * i) * stride] + p[(2 * i + 1) * stride];
  return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

// Per-token codes of the lane's Q rows (rows past T repeat row T-1 and store
// the bytes its owner stores, so no store needs a branch).
__device__ __forceinline__ void quant_span_rows(const uint4 (&raw)[kSlotRows], int64_t r0, int64_t T,
                                                const PoolLane& pl, int64_t b, int h, int H,
                                                int64_t TP, int8_t* __restrict__ qi,
                                                float* __restrict__ qs) {
#pragma unroll
  for (int m = 0; m < kSlotRows; ++m) {
    float x[8];
    unpack8(raw[m], x);
    uint2 codes;
    const float ss = quant_token_row(x, codes);
    const int64_t row = (b * TP + min(r0 + pl.g + 16 * m, T - 1)) * H + h;
    *reinterpret_cast<uint2*>(qi + row * kHeadDim + pl.c8) = codes;
    if (pl.c8 == 0) qs[row] = ss;
    __builtin_amdgcn_sched_barrier(0);  // one row at a time
  }
}

// pool_kernel's row access: raw buffer loads with a wave-uniform base per
// 16-row step and one offset VGPR for all of the lane's rows (in place of a
// 64-bit address each). Rows past T read zeros (or, for a row stride below
// 128 elements, rows the pooling masks out). Row strides are 0 <= st < 2^26.
__device__ __forceinline__ void load_span_buf(const uint16_t* xh, int64_t st, int64_t r0, int64_t T,
                                              const PoolLane& pl, uint4 (&raw)[kSlotRows]) {
  const uint32_t off = static_cast<uint32_t>((pl.g * st + pl.c8) * 2);
  const int64_t cap = max<int64_t>(32 * st, 2 * kHeadDim);
#pragma unroll
  for (int m = 0; m < kSlotRows; ++m) {
    const int64_t rb = r0 + 16 * m;
    raw[m] = buffer_load16(xh + rb * st, rows_nbytes(rb, T, 2 * st, 2 * kHeadDim, cap), off);
  }
}

// Per-token codes of the lane's Q rows; stores of rows past T fall outside the
// range of their buffer store and are dropped.
__device__ __forceinline__ void quant_span_rows_buf(const uint4 (&raw)[kSlotRows], int64_t r0,
                                                    int64_t T, const PoolLane& pl, int64_t b, int h,
                                                    int H, int64_t TP, int8_t* __restrict__ qi,
                                                    float* __restrict__ qs) {
  typedef __attribute__((__vector_size__(2 * sizeof(uint32_t)))) uint32_t u32x2;
  const int64_t pitch = static_cast<int64_t>(H) * kHeadDim;  // bytes per token of qi
  const uint32_t off = static_cast<uint32_t>(pl.g * pitch + pl.c8);
#pragma unroll
  for (int m = 0; m < kSlotRows; ++m) {
    float x[8];
    unpack8(raw[m], x);
    uint2 codes;
    const float ss = quant_token_row(x, codes);
    const int64_t rb = r0 + 16 * m;
    const u32x2 cv = {codes.x, codes.y};
    __builtin_amdgcn_raw_buffer_store_b64(
        cv, buffer_rsrc(qi + ((b * TP + rb) * H + h) * kHeadDim, rows_nbytes(rb, T, pitch, kHeadDim, 16 * pitch)),
        off, 0, 0);
    if (pl.c8 == 0 && rb + pl.g < T) qs[(b * TP + rb + pl.g) * H + h] = ss;
    __builtin_amdgcn_sched_barrier(0);  // one row at a time
  }
}

// QUANT: Q's rows come first and are quantised while K's and V's land, then
// Q, K and V are pooled in that order; otherwise K, V, Q. AMAX: the per-block
// |v| max (vamax_part).
template <int BLK, bool QUANT, bool AMAX>
__global__ void __launch_bounds__(kPoolThreads)
pool_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
            const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
            const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t T,
            int H, int NT, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t npad,
            float* __restrict__ qbar, float* __restrict__ vamax_part, int8_t* __restrict__ qi,
            float* __restrict__ qs, int64_t TP) {
  constexpr int NB = kSpan / BLK;
  __shared__ __align__(16) float part[NB * kSlots * kHeadDim];
  __shared__ __align__(16) float amx[AMAX ? NB * kSlots * kHeadDim : 4];
  const int h = blockIdx.x;
  const int64_t b = blockIdx.z, r0 = static_cast<int64_t>(blockIdx.y) * kSpan;
  const PoolLane pl;
  uint4 rk[kSlotRows], rv[kSlotRows], rq[kSlotRows];
  if (QUANT) load_span_buf(q + b * sq_b + h * sq_h, sq_t, r0, T, pl, rq);
  load_span_buf(k + b * sk_b + h * sk_h, sk_t, r0, T, pl, rk);
  load_span_buf(v + b * sv_b + h * sv_h, sv_t, r0, T, pl, rv);
  if (!QUANT) load_span_buf(q + b * sq_b + h * sq_h, sq_t, r0, T, pl, rq);
  // this thread's output: block s*NB + blk (if it exists), channel c
  const int blk = static_cast<int>(threadIdx.x) >> 7, c = static_cast<int>(threadIdx.x) & 127;
  const int j = static_cast<int>(blockIdx.y) * NB + blk;
  const bool out = blk < NB && j < NT;
  const float flen = static_cast<float>(min<int64_t>(BLK, T - static_cast<int64_t>(j) * BLK));
  const float* pc = part + blk * kSlots * kHeadDim + c;
  const auto pool_q = [&]() {
    pool_span<BLK, false>(rq, r0, T, pl, part, nullptr);
    __syncthreads();
    if (out) qbar[((b * H + h) * NT + j) * kHeadDim + c] = tree16(pc, kHeadDim) / flen;
    __syncthreads();
  };

  if (QUANT) {
    quant_span_rows_buf(rq, r0, T, pl, b, h, H, TP, qi, qs);
    pool_q();
  }
  pool_span<BLK, false>(rk, r0, T, pl, part, nullptr);
  __syncthreads();
  if (out) kc[((b * npad + j) * H + h) * kHeadDim + c] = f2bf(tree16(pc, kHeadDim) / flen);
  __syncthreads();
  pool_span<BLK, AMAX>(rv, r0, T, pl, part, amx);
  __syncthreads();
  if (out) {
    vc[((b * npad + j) * H + h) * kHeadDim + c] = f2bf(tree16(pc, kHeadDim));
    if (AMAX) {
      const float* ac = amx + blk * kSlots * kHeadDim + c;
      float m = ac[0];
#pragma unroll
      for (int g = 1; g < kSlots; ++g) m = fmaxf(m, ac[g * kHeadDim]);
      vamax_part[((b * NT + j) * H + h) * kHeadDim + c] = m;
    }
  }
  if (!QUANT) {
    __syncthreads();
    pool_q();
  }
}

// --------------------------------------------------------------- moments --
// /root/reference/_preprocess.py:241-243 and /root/reference/_fused_prep.py:77-81.
// 8 partial groups sum blocks j = g (mod 8) in ascending order; the partials
// are combined ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)).
template <int N>
__device__ __forceinline__ float tree8(const float (*part)[N], int d) {
  return ((part[0][d] + part[1][d]) + (part[2][d] + part[3][d])) +
         ((part[4][d] + part[5][d]) + (part[6][d] + part[7][d]));
}

// One workgroup of 8 x kMomCh threads per (channel slice, head, batch), kMomCh
// channels a slice: thread t owns partial group g = t / kMomCh (blocks j = g
// mod 8, summed in ascending order) and channel c = slice * kMomCh + t %
// kMomCh. A thread's serial work is one channel and each SIMD holds at most one
// of the launch's waves, so the chains run side by side on 8 CUs per head. A
// thread loads kMomR of its blocks at once (2-byte buffer loads); up to NT = 8
// * kMomR (every block of the head) they stay in registers for the centring
// pass, so the kernel reads kc from HBM once. With vamax_part the same thread
// takes the |v| max of its channel over the same blocks, loaded beside them.
constexpr int kMomCh = 16;
constexpr int kMomThreads = 8 * kMomCh;
constexpr int kMomR = 32;
template <bool CENTRE>
__global__ void __launch_bounds__(kMomThreads)
moments_kernel(uint16_t* __restrict__ kc, int64_t npad, int NT, int H,
               float* __restrict__ kc_mean, float* __restrict__ kc_var,
               const float* __restrict__ vamax_part, float* __restrict__ vscale) {
  const int h = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, g = t / kMomCh, cl = t % kMomCh;
  const int c = static_cast<int>(blockIdx.x) * kMomCh + cl;
  __shared__ float part[8][kMomCh];
  __shared__ float amx[8][kMomCh];
  __shared__ float smean[kMomCh];
  const float fnt = static_cast<float>(NT);
  // Rows through raw buffer loads: per chunk of 8 * kMomR rows from row r, a
  // wave-uniform base at row r and the lane's row g + 8u, channel c at a
  // 32-bit offset (below 2^32 for H < 65536); rows past NT read 0.
  constexpr int kChunk = 8 * kMomR;
  uint16_t* kch = kc + (static_cast<int64_t>(b) * npad * H + h) * kHeadDim;
  const float* ah = vamax_part + (static_cast<int64_t>(b) * NT * H + h) * kHeadDim;
  const int64_t sj = static_cast<int64_t>(H) * kHeadDim;
  const auto koff = [&](int u) { return static_cast<uint32_t>(((g + 8 * u) * sj + c) * 2); };
  const auto kbytes = [&](int64_t r) { return rows_nbytes(r, NT, 2 * sj, 2 * kHeadDim, kChunk * 2 * sj); };
  const auto abytes = [&](int64_t r) { return rows_nbytes(r, NT, 4 * sj, 4 * kHeadDim, kChunk * 4 * sj); };
  const bool resident = NT <= kChunk;
  uint16_t w[kMomR];
  float s = 0.f, am = 0.f;
  for (int r = 0; r < NT; r += kChunk) {  // this thread's rows r + g + 8u
    const uint32_t kb = kbytes(r);
#pragma unroll
    for (int u = 0; u < kMomR; ++u) w[u] = buffer_load2(kch + r * sj, kb, koff(u));
    if (vamax_part) {
      const uint32_t ab = abytes(r);
      float a[kMomR];
#pragma unroll
      for (int u = 0; u < kMomR; ++u)
        a[u] = __uint_as_float(buffer_load4(ah + r * sj, ab, 2 * koff(u)));
#pragma unroll
      for (int u = 0; u < kMomR; ++u) am = fmaxf(am, a[u]);  // rows past NT read 0
    }
#pragma unroll
    for (int u = 0; u < kMomR; ++u)
      if (r + g + 8 * u < NT) s = s + bf2f(w[u]);
  }
  part[g][cl] = s;
  amx[g][cl] = am;
  __syncthreads();
  const int64_t mo = (static_cast<int64_t>(b) * H + h) * kHeadDim + c;
  if (t < kMomCh) {
    const float mean = tree8(part, t) / fnt;
    smean[t] = mean;
    kc_mean[mo] = mean;
  } else if (vamax_part && t < 2 * kMomCh) {
    const int d = t - kMomCh;
    float m = amx[0][d];
    for (int i = 1; i < 8; ++i) m = fmaxf(m, amx[i][d]);
    // absmax.div(127.0) in torch is a multiply by the fp32 reciprocal
    // (/root/reference/_fused_quant.py:104).
    const float sc = m * (1.0f / 127.0f);
    vscale[mo] = sc < 1e-8f ? 1e-8f : sc;  // c = slice * kMomCh + d
  }
  __syncthreads();
  const float mean = smean[cl];
  float acc = 0.f;
  for (int r = 0; r < NT; r += kChunk) {
    const uint32_t kb = kbytes(r);
    if (!resident) {
#pragma unroll
      for (int u = 0; u < kMomR; ++u) w[u] = buffer_load2(kch + r * sj, kb, koff(u));
    }
#pragma unroll
    for (int u = 0; u < kMomR; ++u) {
      if (r + g + 8 * u < NT) {
        float y = bf2f(w[u]) - mean;
        if (CENTRE) {  // bf16 of the centred value (round to nearest even, as f2bf)
          const uint16_t nb = static_cast<uint16_t>(cvt_pk_bf16(y, 0.f));
          y = bf2f(nb);
          buffer_store2(kch + r * sj, kb, koff(u), nb);
        }
        acc = acc + y * y;
      }
    }
  }
  __syncthreads();  // every thread has read part[] above
  part[g][cl] = acc;
  __syncthreads();
  if (t < kMomCh) kc_var[mo] = tree8(part, t) / fnt;
}

// ------------------------------------------------------ single-read INT8 --
// The INT8 path's preparation with one read of Q, K and V
// (/root/reference/_fused_prep.py:62-98 reads K and V twice). A head's K codes
// need the mean of all its pooled keys and its V codes the per-channel |max|
// over all its tokens, so a workgroup keeps its K and V rows in registers
// across two barriers over the workgroups of that head:
//   phase 1  load the span's Q, K and V rows; quantise and pool Q, pool K and
//            V (as pool_kernel: same partials, same outputs, |v| max per block)
//   barrier
//   phase 2  16 workgroups, one per 8-channel slice: kc mean, centred kc, kc
//            variance and V scale of the head (moments_kernel's order)
//   barrier
//   phase 3  K codes (smoothed by the mean, per token) and V codes (per
//            channel) from the rows still in registers.
// The grid is launched cooperatively (every workgroup resident) as teams of
// S = ceil(T / 128) workgroups; team t handles heads t, t + nteams, ..., so
// one team's VALU phases overlap another's loads. A team's barrier counter
// (sync[1 + team], zeroed by sync_init_kernel) counts arrivals; barrier n of a
// head waits for n * S of them. The wait is bounded: a barrier not met within
// ~0.1 s sets sync[0] and releases its waiter, so no schedule can hang the
// device (with every workgroup resident, each arrives and the bound is never
// met).
constexpr int kMomSlices = kHeadDim / 8;  // 8-channel slices of the moments phase
constexpr uint32_t kSpinLimit = 1u << 21; // ~0.1 s of 128-cycle sleeps

__global__ void sync_init_kernel(uint32_t* __restrict__ sync, int n) {
  for (int i = threadIdx.x; i < n; i += blockDim.x) sync[i] = 0u;
}

// Values one workgroup hands to another inside the launch (pooled keys, |v|
// maxima, the mean and the V scale) move through relaxed device-scope atomic
// loads and stores, which write through / read past the XCDs' non-coherent
// L2s; nothing else needs to be visible before the launch ends, so the
// barrier itself flushes no cache (a device-scope fence writes back and
// invalidates a whole L2, and one per wave at every barrier cost ~0.15 ms).
__device__ __forceinline__ void xstore(uint32_t* p, uint32_t v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint32_t xload(const uint32_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ uint64_t xload64(const uint64_t* p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Every thread's stores have completed (s_waitcnt 0) before the workgroup
// arrives; the counter and the poll are device-scope atomics.
__device__ __forceinline__ void team_barrier(uint32_t* ctr, uint32_t target, uint32_t* err) {
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    uint32_t spins = 0;
    while (xload(ctr) < target) {
      if (++spins > kSpinLimit) {
        xstore(err, 1u);
        break;
      }
      __builtin_amdgcn_s_sleep(2);
    }
  }
  __syncthreads();
}

// Moments of channels [8cs, 8cs + 8) of head (b, h), in moments_kernel's order:
// 8 partials over blocks j = g (mod 8) ascending, tree8; kc centred in place
// (bf16), variance of the centred values; vscale from the per-block |v| max.
// skc: NT x 8 fp32 of dynamic LDS; red: 32 fp32 of LDS.
__device__ __forceinline__ void moments_slice(uint16_t* __restrict__ kc, int64_t npad,
                                              const float* __restrict__ vamax_part,
                                              float* __restrict__ kc_mean,
                                              float* __restrict__ kc_var,
                                              float* __restrict__ vscale, int64_t b, int h, int H,
                                              int NT, int cs, float* skc, float* red) {
  __shared__ float psum[8][8];
  __shared__ float smean[8];
  const int t = threadIdx.x;
  const int64_t sj = static_cast<int64_t>(H) * kHeadDim;
  uint16_t* col = kc + (b * npad * H + h) * kHeadDim + 8 * cs;
  float am[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j = t; j < NT; j += kPoolThreads) {
    const uint64_t* kr = reinterpret_cast<const uint64_t*>(col + j * sj);
    const uint64_t w0 = xload64(kr), w1 = xload64(kr + 1);
    float x[8];
    unpack8(make_uint4(static_cast<uint32_t>(w0), static_cast<uint32_t>(w0 >> 32),
                       static_cast<uint32_t>(w1), static_cast<uint32_t>(w1 >> 32)), x);
    float4* d = reinterpret_cast<float4*>(skc + 8 * j);
    d[0] = make_float4(x[0], x[1], x[2], x[3]);
    d[1] = make_float4(x[4], x[5], x[6], x[7]);
    if (vamax_part) {
      const uint64_t* ar = reinterpret_cast<const uint64_t*>(
          vamax_part + ((b * NT + j) * H + h) * kHeadDim + 8 * cs);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint64_t w = xload64(ar + i);
        am[2 * i] = fmaxf(am[2 * i], __uint_as_float(static_cast<uint32_t>(w)));
        am[2 * i + 1] = fmaxf(am[2 * i + 1], __uint_as_float(static_cast<uint32_t>(w >> 32)));
      }
    }
  }
  if (vamax_part) {
    // max over the wave (any order: max is exact), then over the 4 waves
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int o = 32; o >= 1; o >>= 1) am[e] = fmaxf(am[e], __shfl_xor(am[e], o));
    if ((t & 63) == 0)
#pragma unroll
      for (int e = 0; e < 8; ++e) red[8 * (t >> 6) + e] = am[e];
  }
  __syncthreads();
  const int g = t >> 3, e = t & 7;  // threads t < 64: partial g, channel e
  if (t < 64) {
    float acc = 0.f;
#pragma unroll 8
    for (int j = g; j < NT; j += 8) acc = acc + skc[8 * j + e];
    psum[g][e] = acc;
  }
  __syncthreads();
  const int64_t mo = (b * H + h) * kHeadDim + 8 * cs;
  if (t < 8) {
    const float mean = (((psum[0][t] + psum[1][t]) + (psum[2][t] + psum[3][t])) +
                        ((psum[4][t] + psum[5][t]) + (psum[6][t] + psum[7][t]))) /
                       static_cast<float>(NT);
    smean[t] = mean;
    xstore(reinterpret_cast<uint32_t*>(kc_mean + mo + t), __float_as_uint(mean));
    if (vamax_part) {
      const float m = fmaxf(fmaxf(red[t], red[8 + t]), fmaxf(red[16 + t], red[24 + t]));
      const float sc = m * (1.0f / 127.0f);  // torch's scalar divide: a multiply by 1/127
      xstore(reinterpret_cast<uint32_t*>(vscale + mo + t), __float_as_uint(sc < 1e-8f ? 1e-8f : sc));
    }
  }
  __syncthreads();
  for (int j = t; j < NT; j += kPoolThreads) {
    uint16_t nb[8];
#pragma unroll
    for (int c = 0; c < 8; ++c) {
      nb[c] = f2bf(skc[8 * j + c] - smean[c]);
      const float y = bf2f(nb[c]);
      skc[8 * j + c] = y * y;
    }
    *reinterpret_cast<uint4*>(col + j * sj) =
        make_uint4(nb[0] | (static_cast<uint32_t>(nb[1]) << 16), nb[2] | (static_cast<uint32_t>(nb[3]) << 16),
                   nb[4] | (static_cast<uint32_t>(nb[5]) << 16), nb[6] | (static_cast<uint32_t>(nb[7]) << 16));
  }
  __syncthreads();
  if (t < 64) {
    float acc = 0.f;
#pragma unroll 8
    for (int j = g; j < NT; j += 8) acc = acc + skc[8 * j + e];
    psum[g][e] = acc;
  }
  __syncthreads();
  if (t < 8)
    kc_var[mo + t] = (((psum[0][t] + psum[1][t]) + (psum[2][t] + psum[3][t])) +
                      ((psum[4][t] + psum[5][t]) + (psum[6][t] + psum[7][t]))) /
                     static_cast<float>(NT);
  __syncthreads();  // skc, red and psum are reused
}

struct PrepInt8Args {
  const uint16_t *q, *k, *v;
  int64_t sq_b, sq_t, sq_h, sk_b, sk_t, sk_h, sv_b, sv_t, sv_h;
  int64_t T, TP, npad;
  int B, H, NT, S, nteams;
  uint16_t *kc, *vc;
  float *qbar, *kc_mean, *kc_var, *vscale, *vamax_part;  // vscale, vamax_part: null without V codes
  int8_t *qi, *ki, *vi;
  float *qs, *ks;
  int64_t ks_st, ks_sh;  // element strides of ks within a batch's TP*H scales
  uint32_t* sync;        // the bound flag, then nteams barrier counters
};

template <int BLK, bool PV>
__global__ void __launch_bounds__(kPoolThreads) __attribute__((amdgpu_waves_per_eu(2)))
prep_int8_single_read_kernel(const PrepInt8Args a) {
  constexpr int NB = kSpan / BLK;
  __shared__ __align__(16) float part[NB * kSlots * kHeadDim];
  __shared__ __align__(16) float amx[NB * kSlots * kHeadDim];
  extern __shared__ __align__(16) float skc_lds[];  // NT x 8 (moments phase)
  const int team = static_cast<int>(blockIdx.x) / a.S, s = static_cast<int>(blockIdx.x) % a.S;
  uint32_t* err = a.sync;
  uint32_t* ctr = a.sync + 1 + team;
  const int64_t r0 = static_cast<int64_t>(s) * kSpan, T = a.T;
  const int H = a.H, NT = a.NT;
  const PoolLane pl0;
  const int blk = static_cast<int>(threadIdx.x) >> 7, c = static_cast<int>(threadIdx.x) & 127;
  const int j = s * NB + blk;
  const bool out = blk < NB && j < NT;
  const float flen = static_cast<float>(min<int64_t>(BLK, T - static_cast<int64_t>(j) * BLK));
  const float* pc = part + blk * kSlots * kHeadDim + c;
  // the exchange stores go by channel pairs: thread t, block t / 64, channels
  // 2(t % 64) and 2(t % 64) + 1
  const int blk2 = static_cast<int>(threadIdx.x) >> 6, c2 = 2 * (static_cast<int>(threadIdx.x) & 63);
  const int j2 = s * NB + blk2;
  const bool out2 = blk2 < NB && j2 < NT;
  const float flen2 = static_cast<float>(min<int64_t>(BLK, T - static_cast<int64_t>(j2) * BLK));
  const float* pc2 = part + blk2 * kSlots * kHeadDim + c2;
  uint32_t epoch = 0;
  const int BH = a.B * H;
  for (int bh = team; bh < BH; bh += a.nteams) {
    const int64_t b = bh / H;
    const int h = bh % H;
    // The lane's row offsets do not change from head to head; left visible,
    // the compiler keeps all of them (64-bit each) live across the loop and
    // spills them. Through the empty asm they are recomputed per head.
    PoolLane pl = pl0;
    asm volatile("" : "+v"(pl.g));
    // ---- phase 1: one read of the span's rows (Q's are processed while K's
    // and V's land)
    uint4 rq[kSlotRows], rk[kSlotRows], rv[kSlotRows];
    load_span(a.q + b * a.sq_b + h * a.sq_h + pl.c8, a.sq_t, r0, T, pl.g, rq);
    load_span(a.k + b * a.sk_b + h * a.sk_h + pl.c8, a.sk_t, r0, T, pl.g, rk);
    load_span(a.v + b * a.sv_b + h * a.sv_h + pl.c8, a.sv_t, r0, T, pl.g, rv);
    quant_span_rows(rq, r0, T, pl, b, h, H, a.TP, a.qi, a.qs);
    pool_span<BLK, false>(rq, r0, T, pl, part, nullptr);
    __syncthreads();
    if (out) a.qbar[((b * H + h) * NT + j) * kHeadDim + c] = tree16(pc, kHeadDim) / flen;
    __syncthreads();
    pool_span<BLK, false>(rk, r0, T, pl, part, nullptr);
    __syncthreads();
    if (out2)  // read by another workgroup in phase 2: an exchange store
      xstore(reinterpret_cast<uint32_t*>(a.kc + ((b * a.npad + j2) * H + h) * kHeadDim + c2),
             pack_bf16x2(tree16(pc2, kHeadDim) / flen2, tree16(pc2 + 1, kHeadDim) / flen2));
    __syncthreads();
    pool_span<BLK, PV>(rv, r0, T, pl, part, amx);
    __syncthreads();
    if (out) a.vc[((b * a.npad + j) * H + h) * kHeadDim + c] = f2bf(tree16(pc, kHeadDim));
    if (PV && out2) {
      const float* ac = amx + blk2 * kSlots * kHeadDim + c2;
      float m0 = ac[0], m1 = ac[1];
#pragma unroll
      for (int g = 1; g < kSlots; ++g) {
        m0 = fmaxf(m0, ac[g * kHeadDim]);
        m1 = fmaxf(m1, ac[g * kHeadDim + 1]);
      }
      uint32_t* d = reinterpret_cast<uint32_t*>(a.vamax_part + ((b * NT + j2) * H + h) * kHeadDim + c2);
      xstore(d, __float_as_uint(m0));
      xstore(d + 1, __float_as_uint(m1));
    }
    team_barrier(ctr, ++epoch * static_cast<uint32_t>(a.S), err);
    // ---- phase 2: the head's moments, one 8-channel slice per workgroup
    for (int cs = s; cs < kMomSlices; cs += a.S)
      moments_slice(a.kc, a.npad, PV ? a.vamax_part : nullptr, a.kc_mean, a.kc_var, a.vscale, b,
                    h, H, NT, cs, skc_lds, part);
    team_barrier(ctr, ++epoch * static_cast<uint32_t>(a.S), err);
    // ---- phase 3: K and V codes from the rows in registers
    const int64_t mo = (b * H + h) * kHeadDim + pl.c8;
    float mean[8], sv[8], rr[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {  // written by the phase-2 workgroups
      mean[e] = __uint_as_float(xload(reinterpret_cast<const uint32_t*>(a.kc_mean + mo + e)));
      sv[e] = PV ? __uint_as_float(xload(reinterpret_cast<const uint32_t*>(a.vscale + mo + e))) : 1.f;
      rr[e] = __builtin_amdgcn_rcpf(sv[e]);
    }
#pragma unroll
    for (int m = 0; m < kSlotRows; ++m) {
      // rows past T repeat row T-1 and store what its owner stores
      const int64_t t = min(r0 + pl.g + 16 * m, T - 1);
      const int64_t row = (b * a.TP + t) * H + h;
      float x[8], y[8];
      unpack8(rk[m], x);
#pragma unroll
      for (int e = 0; e < 8; ++e) y[e] = x[e] - mean[e];
      uint2 codes;
      const float ss = quant_token_row(y, codes);
      *reinterpret_cast<uint2*>(a.ki + row * kHeadDim + pl.c8) = codes;
      if (pl.c8 == 0) a.ks[b * a.TP * H + t * a.ks_st + h * a.ks_sh] = ss;
      if (PV) {
        unpack8(rv[m], x);
        *reinterpret_cast<uint2*>(a.vi + row * kHeadDim + pl.c8) = codes8(x, rr, sv);
      }
      __builtin_amdgcn_sched_barrier(0);  // one row at a time: registers stay at one row's
    }
  }
}

// ----------------------------------------------------------------- route --
// Thresholds (/root/reference/_preprocess.py:149-163, /root/reference/_fused_prep.py:50-59)
// and the routing rule of the forward (/root/reference/_tri_fwd.py:279-286),
// for kQB query blocks per workgroup.
constexpr int kQB = 8;
constexpr int kRouteThreads = 256;
constexpr int kMaxWords = 512;  // NT <= 16384 (the forwards' limit)
// The workgroup's threads form G groups of R = kRouteThreads / G (a multiple
// of 64: whole waves); thread t scores key block (kc row) j0 + t % R against
// the kQB / G query blocks of its group, its row streaming through registers
// 32 channels at a time (the next 32 in flight); the query centroids are
// wave-uniform, so each fma takes its q operand from an SGPR (scalar loads).
// G > 1 serves short sequences (NT <= 128), whose rows would leave waves idle.
// Against kc rows staged in LDS with two or four threads per row: 20.0 ->
// 19.7 us at NT 256 and 63.0 -> 47.2 us at NT 512, same bits.
template <int G>
__global__ void __launch_bounds__(kRouteThreads)
route_kernel(const float* __restrict__ qbar, const uint16_t* __restrict__ kc, int64_t npad,
             const float* __restrict__ kc_mean, const float* __restrict__ kc_var, int H, int NT,
             int W, float c, float c2, float tau, int mode, int64_t skv_lo, int64_t skv_hi,
             int64_t sq_lo, int64_t sq_hi, float* __restrict__ thr_out,
             int32_t* __restrict__ counts, uint32_t* __restrict__ mask) {
  const int i0 = blockIdx.x * kQB, h = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  extern __shared__ __align__(16) uint32_t smask_lds[];
  const auto smask = [&](int i, int w) -> uint32_t& { return smask_lds[i * W + w]; };
  __shared__ __align__(16) float sq[kQB][kHeadDim];  // the kQB query centroids
  __shared__ __align__(16) float smk[kHeadDim];      // kc mean (mode 0)
  __shared__ __align__(16) float svk[kHeadDim];      // kc variance
  static_assert(kQB * kHeadDim / 4 == kRouteThreads && 2 * kHeadDim == kRouteThreads,
                "one float4 of the centroids and one moment per thread");
  const int64_t bh = static_cast<int64_t>(b) * H + h;
  {
    // The centroids and moments, one load per thread. Query rows past NT (a
    // ragged last workgroup) read row NT-1; nothing of theirs is stored.
    const int qb = t >> 5, q4 = t & 31;
    const float4 x =
        reinterpret_cast<const float4*>(qbar + (bh * NT + min(i0 + qb, NT - 1)) * kHeadDim)[q4];
    const float mv = t < kHeadDim ? kc_mean[bh * kHeadDim + t] : kc_var[bh * kHeadDim + t - kHeadDim];
    reinterpret_cast<float4*>(&sq[qb][0])[q4] = x;
    (t < kHeadDim ? smk[t] : svk[t - kHeadDim]) = mv;
  }
  for (int e = t; e < kQB * W; e += kRouteThreads) smask_lds[e] = 0u;
  constexpr int R = kRouteThreads / G, kQG = kQB / G;  // rows per pass, query blocks per thread
  static_assert(R % 64 == 0 && kQB % G == 0, "route groups are whole waves");
  const int rr = t % R;
  const int ig = __builtin_amdgcn_readfirstlane(t / R) * kQG;  // the group's first query block
  const float* qrow[kQG];  // wave-uniform rows of the centroids
#pragma unroll
  for (int i = 0; i < kQG; ++i) qrow[i] = qbar + (bh * NT + min(i0 + ig + i, NT - 1)) * kHeadDim;
  // kc rows through raw buffer loads: base at row j0 (wave-uniform), the lane's
  // row rr further; rows past NT read 0 (and are not active).
  const uint16_t* kch = kc + (static_cast<int64_t>(b) * npad * H + h) * kHeadDim;
  const int64_t sj = static_cast<int64_t>(H) * kHeadDim;
  const uint32_t roff = static_cast<uint32_t>(rr * sj * 2);
  __syncthreads();  // the centroids, moments and cleared mask words
  // Every wave computes the kQB thresholds (lane i: query block i0 + i), one
  // fma chain per moment in ascending d, so no barrier waits on them.
  float th;
  {
    const float* qv = sq[min(lane, kQB - 1)];
    float mu = 0.f, var = 0.f;
#pragma unroll 4
    for (int d = 0; d < kHeadDim; d += 4) {
      const float4 x = *reinterpret_cast<const float4*>(qv + d);
      const float4 vk = *reinterpret_cast<const float4*>(svk + d);
      if (mode == 0) {
        const float4 mk = *reinterpret_cast<const float4*>(smk + d);
        mu = fmaf(x.x, mk.x, mu);
        var = fmaf(x.x * x.x, vk.x, var);
        mu = fmaf(x.y, mk.y, mu);
        var = fmaf(x.y * x.y, vk.y, var);
        mu = fmaf(x.z, mk.z, mu);
        var = fmaf(x.z * x.z, vk.z, var);
        mu = fmaf(x.w, mk.w, mu);
        var = fmaf(x.w * x.w, vk.w, var);
      } else {
        var = fmaf(x.x * x.x, vk.x, var);
        var = fmaf(x.y * x.y, vk.y, var);
        var = fmaf(x.z * x.z, vk.z, var);
        var = fmaf(x.w * x.w, vk.w, var);
      }
    }
    if (mode == 0) {
      mu = mu * c;
      var = var * c2;
      const float sd = sqrtf(fmaxf(var, 0.f) + 1e-6f);
      th = mu + tau * sd;
    } else {
      var = var * c2;
      th = tau * sqrtf(var + 1e-6f);
    }
    if (wave == 0 && lane < kQB && i0 + lane < NT)
      thr_out[(static_cast<int64_t>(b) * NT + i0 + lane) * H + h] = th;
  }
  constexpr int kCh = 32;                  // channels of the row per step
  constexpr int kChLoads = kCh / 8;        // 16-byte loads per step
  for (int j0 = 0; j0 < NT; j0 += R) {
    const int j = j0 + rr;
    const bool active = j < NT;
    const uint16_t* base = kch + j0 * sj;
    const uint32_t nb = rows_nbytes(j0, NT, 2 * sj, 2 * kHeadDim, R * 2 * sj);
    float acc[kQG];
#pragma unroll
    for (int i = 0; i < kQG; ++i) acc[i] = 0.f;
    uint4 kn[kChLoads];  // the next channel step of this thread's row, in flight
#pragma unroll
    for (int u = 0; u < kChLoads; ++u) kn[u] = buffer_load16(base, nb, roff + 16 * u);
#pragma unroll 1
    for (int d0 = 0; d0 < kHeadDim; d0 += kCh) {
      uint4 kr[kChLoads];
#pragma unroll
      for (int u = 0; u < kChLoads; ++u) kr[u] = kn[u];
      if (d0 + kCh < kHeadDim) {
#pragma unroll
        for (int u = 0; u < kChLoads; ++u)
          kn[u] = buffer_load16(base, nb, roff + 2 * (d0 + kCh) + 16 * u);
      }
#pragma unroll
      for (int d4 = 0; d4 < kCh / 4; ++d4) {
        const uint4& w = kr[d4 / 2];
        const uint32_t k01 = (d4 & 1) ? w.z : w.x, k23 = (d4 & 1) ? w.w : w.y;
        const float k0 = lo_bf16(k01), k1 = hi_bf16(k01), k2 = lo_bf16(k23), k3 = hi_bf16(k23);
#pragma unroll
        for (int i = 0; i < kQG; ++i) {
          const float4 qv = *reinterpret_cast<const float4*>(qrow[i] + d0 + 4 * d4);
          acc[i] = fmaf(qv.x, k0, acc[i]);
          acc[i] = fmaf(qv.y, k1, acc[i]);
          acc[i] = fmaf(qv.z, k2, acc[i]);
          acc[i] = fmaf(qv.w, k3, acc[i]);
        }
      }
    }
    const bool in_skv = j >= skv_lo && j < skv_hi;
    const int w0 = (j0 + 64 * (wave % (R / 64))) >> 5;  // this wave's 64 rows
#pragma unroll
    for (int i = 0; i < kQG; ++i) {
      const int il = ig + i;
      const int qi = i0 + il;
      const float r = acc[i] * c;
      const int dij = qi > j ? qi - j : j - qi;
      const bool q_in_sink = qi >= sq_lo && qi < sq_hi;
      const float thr = __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, th), il));
      const bool routed = (r > thr) || dij <= 1 || in_skv;
      const bool exact = active && qi < NT && (q_in_sink || routed);
      const uint64_t bal = __ballot(exact);
      if (lane == 0 && w0 < W) {
        smask(il, w0) = static_cast<uint32_t>(bal);
        if (w0 + 1 < W) smask(il, w0 + 1) = static_cast<uint32_t>(bal >> 32);
      }
    }
  }
  __syncthreads();

  // Masks and exact-block counts, one query block per wave at a time.
  for (int i = wave; i < kQB; i += kRouteThreads / 64) {
    const int qi = i0 + i;
    if (qi >= NT) break;
    const int64_t row = bh * NT + qi;
    int base = 0;
    for (int w0 = 0; w0 < W; w0 += 64) {
      const int w = w0 + lane;
      const uint32_t word = w < W ? smask(i, w) : 0u;
      if (w < W) mask[row * W + w] = word;
      int cnt = __popc(word);
#pragma unroll
      for (int s = 32; s >= 1; s >>= 1) cnt += __shfl_xor(cnt, s);
      base += cnt;
    }
    if (lane == 0) counts[row] = base;
  }
}

}  // namespace solattn

using namespace solattn;

namespace {

int check_bthd(const void* p, int64_t sb, int64_t st, int64_t sh, const char* name) {
  SOLATTN_REQUIRE(p != nullptr, SOLATTN_EINVAL, "%s: null pointer", name);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(p) % 16 == 0 && sb % 8 == 0 && st % 8 == 0 &&
                      sh % 8 == 0,
                  SOLATTN_EINVAL,
                  "%s: base must be 16-byte aligned and strides multiples of 8 elements", name);
  return 0;
}

}  // namespace

namespace solattn {

int launch_pool(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t* k,
                int64_t sk_b, int64_t sk_t, int64_t sk_h, const uint16_t* v, int64_t sv_b,
                int64_t sv_t, int64_t sv_h, int64_t B, int64_t T, int64_t H, int64_t block,
                uint16_t* kc, uint16_t* vc, int64_t npad, float* qbar, float* vamax_part,
                int8_t* qi, float* qs, int64_t TP, hipStream_t s) {
  const int64_t NT = cdiv(T, block);
  const int64_t spans = cdiv(T, kSpan);
  SOLATTN_REQUIRE(spans <= 65535 && B <= 65535 && H <= 65535, SOLATTN_EUNSUPPORTED,
                  "pool: %lld tokens x %lld heads x %lld batch", (long long)T, (long long)H,
                  (long long)B);
  SOLATTN_REQUIRE(!qi || (qs && TP >= T && reinterpret_cast<uintptr_t>(qi) % 8 == 0),
                  SOLATTN_EINVAL, "pool: bad Q quantisation outputs");
  SOLATTN_REQUIRE(sq_t >= 0 && sk_t >= 0 && sv_t >= 0 &&
                      std::max(sq_t, std::max(sk_t, sv_t)) < (1ll << 26),
                  SOLATTN_EUNSUPPORTED, "pool: token strides must lie in [0, 2^26)");
  // heads fastest, so the workgroups in flight read whole token rows (all heads)
  // of neighbouring spans
  dim3 grid(static_cast<uint32_t>(H), static_cast<uint32_t>(spans), static_cast<uint32_t>(B));
  const bool amax = vamax_part != nullptr;
  const auto kern =
      block == 64
          ? (qi ? (amax ? pool_kernel<64, true, true> : pool_kernel<64, true, false>)
                : (amax ? pool_kernel<64, false, true> : pool_kernel<64, false, false>))
          : (qi ? (amax ? pool_kernel<128, true, true> : pool_kernel<128, true, false>)
                : (amax ? pool_kernel<128, false, true> : pool_kernel<128, false, false>));
  hipLaunchKernelGGL(kern, grid, dim3(kPoolThreads), 0, s, q, sq_b, sq_t, sq_h, k, sk_b, sk_t,
                     sk_h, v, sv_b, sv_t, sv_h, T, static_cast<int>(H), static_cast<int>(NT), kc,
                     vc, npad, qbar, vamax_part, qi, qs, TP);
  return check_launch("pool");
}

}  // namespace solattn

namespace solattn {

int pool_checked(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t* k,
                 int64_t sk_b, int64_t sk_t, int64_t sk_h, const uint16_t* v, int64_t sv_b,
                 int64_t sv_t, int64_t sv_h, int64_t B, int64_t T, int64_t H, int64_t D,
                 int64_t block, uint16_t* kc, uint16_t* vc, int64_t npad, float* qbar,
                 float* vamax_part, int8_t* qi, float* qs, int64_t TP, hipStream_t s) {
  SOLATTN_REQUIRE(D == kHeadDim, SOLATTN_EUNSUPPORTED, "pool: head_dim %lld != 128", (long long)D);
  SOLATTN_REQUIRE(block == 64 || block == 128, SOLATTN_EUNSUPPORTED, "pool: block %lld not in {64, 128}",
                  (long long)block);
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && B <= 65535 && H <= 65535, SOLATTN_EINVAL,
                  "pool: bad sizes B=%lld T=%lld H=%lld", (long long)B, (long long)T, (long long)H);
  const int64_t NT = cdiv(T, block);
  SOLATTN_REQUIRE(npad >= NT && NT < (1ll << 31), SOLATTN_EINVAL, "pool: npad %lld < NT %lld",
                  (long long)npad, (long long)NT);
  SOLATTN_REQUIRE(kc && vc && qbar, SOLATTN_EINVAL, "pool: null output");
  if (int rc = check_bthd(q, sq_b, sq_t, sq_h, "pool q")) return rc;
  if (int rc = check_bthd(k, sk_b, sk_t, sk_h, "pool k")) return rc;
  if (int rc = check_bthd(v, sv_b, sv_t, sv_h, "pool v")) return rc;
  return launch_pool(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B, T, H, block,
                     kc, vc, npad, qbar, vamax_part, qi, qs, TP, s);
}

}  // namespace solattn

extern "C" int solattn_pool(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                            const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                            const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                            int64_t T, int64_t H, int64_t D, int64_t block, uint16_t* kc,
                            uint16_t* vc, int64_t npad, float* qbar, float* vamax_part,
                            solattn_stream_t stream) {
  clear_error();
  return pool_checked(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B, T, H, D,
                      block, kc, vc, npad, qbar, vamax_part, nullptr, nullptr, 0,
                      reinterpret_cast<hipStream_t>(stream));
}

extern "C" int solattn_moments(uint16_t* kc, int64_t npad, int64_t B, int64_t NT, int64_t H,
                               int64_t D, int centre, float* kc_mean, float* kc_var,
                               const float* vamax_part, float* vscale, solattn_stream_t stream) {
  clear_error();
  SOLATTN_REQUIRE(D == kHeadDim, SOLATTN_EUNSUPPORTED, "moments: head_dim %lld != 128",
                  (long long)D);
  SOLATTN_REQUIRE(B > 0 && NT > 0 && H > 0 && npad >= NT && B <= 65535 && H <= 65535 &&
                      NT < (1ll << 31),
                  SOLATTN_EINVAL, "moments: bad sizes");
  SOLATTN_REQUIRE(kc && kc_mean && kc_var, SOLATTN_EINVAL, "moments: null pointer");
  SOLATTN_REQUIRE(!vamax_part || vscale, SOLATTN_EINVAL, "moments: vamax_part needs vscale");
  SOLATTN_REQUIRE(!vamax_part || H < 32768, SOLATTN_EUNSUPPORTED,
                  "moments: %lld heads with vamax_part (at most 32767)", (long long)H);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(kc) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(vamax_part) % 16 == 0,
                  SOLATTN_EINVAL, "moments: kc and vamax_part must be 16-byte aligned");
  hipLaunchKernelGGL(centre ? moments_kernel<true> : moments_kernel<false>,
                     dim3(kHeadDim / kMomCh, static_cast<uint32_t>(H), static_cast<uint32_t>(B)),
                     dim3(kMomThreads),
                     0, reinterpret_cast<hipStream_t>(stream), kc, npad, static_cast<int>(NT),
                     static_cast<int>(H), kc_mean, kc_var, vamax_part, vscale);
  return check_launch("moments");
}

extern "C" int solattn_route(const float* qbar, const uint16_t* kc, int64_t npad,
                             const float* kc_mean, const float* kc_var, int64_t B, int64_t T,
                             int64_t H, int64_t D, int64_t block, float scale, float tau, int mode,
                             int64_t sink_kv_lo, int64_t sink_kv_hi, int64_t sink_q_lo,
                             int64_t sink_q_hi, float* thr, int32_t* counts, uint32_t* mask,
                             solattn_stream_t stream) {
  clear_error();
  SOLATTN_REQUIRE(D == kHeadDim, SOLATTN_EUNSUPPORTED, "route: head_dim %lld != 128", (long long)D);
  SOLATTN_REQUIRE(block > 0 && B > 0 && T > 0 && H > 0 && B <= 65535 && H <= 65535,
                  SOLATTN_EINVAL, "route: bad sizes");
  const int64_t NT = cdiv(T, block);
  const int64_t W = cdiv(NT, 32);
  SOLATTN_REQUIRE(W <= kMaxWords, SOLATTN_EUNSUPPORTED, "route: %lld blocks exceed %d",
                  (long long)NT, kMaxWords * 32);
  SOLATTN_REQUIRE(npad >= NT, SOLATTN_EINVAL, "route: npad < NT");
  SOLATTN_REQUIRE(mode == 0 || mode == 1, SOLATTN_EINVAL, "route: mode %d", mode);
  SOLATTN_REQUIRE(qbar && kc && kc_var && (mode == 1 || kc_mean) && thr && counts && mask,
                  SOLATTN_EINVAL, "route: null pointer");
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(kc) % 16 == 0, SOLATTN_EINVAL,
                  "route: kc must be 16-byte aligned");
  const float c = scale * kLog2e;
  const float c2 = c * c;
  dim3 grid(static_cast<uint32_t>(cdiv(NT, kQB)), static_cast<uint32_t>(H),
            static_cast<uint32_t>(B));
  hipLaunchKernelGGL(NT <= 64 ? route_kernel<4> : NT <= 128 ? route_kernel<2> : route_kernel<1>,
                     grid, dim3(kRouteThreads),
                     static_cast<size_t>(kQB * W * sizeof(uint32_t)),
                     reinterpret_cast<hipStream_t>(stream), qbar, kc, npad,
                     mode == 0 ? kc_mean : kc_var, kc_var, static_cast<int>(H),
                     static_cast<int>(NT), static_cast<int>(W), c, c2, tau, mode, sink_kv_lo,
                     sink_kv_hi, sink_q_lo, sink_q_hi, thr, counts, mask);
  return check_launch("route");
}

namespace solattn {

int64_t single_read_sync_words(int64_t B, int64_t H) { return B * H + 1; }

namespace {

template <int BLK, bool PV>
const void* single_read_kernel() {
  return reinterpret_cast<const void*>(&prep_int8_single_read_kernel<BLK, PV>);
}

// Teams of the single-read schedule that the device holds at once (every
// workgroup resident), or 0 when fewer than two teams fit: one team would run
// its phases back to back with nothing to overlap them.
int single_read_teams(int64_t B, int64_t T, int64_t H, int64_t block, bool pv, size_t lds) {
  const int64_t S = cdiv(T, kSpan);
  const void* kern = block == 64 ? (pv ? single_read_kernel<64, true>() : single_read_kernel<64, false>())
                                 : (pv ? single_read_kernel<128, true>() : single_read_kernel<128, false>());
  int dev = 0, cus = 0, per_cu = 0;
  if (hipGetDevice(&dev) != hipSuccess ||
      hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
      hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kern, kPoolThreads, lds) != hipSuccess) {
    (void)hipGetLastError();
    return 0;
  }
  const int64_t teams = std::min<int64_t>(B * H, static_cast<int64_t>(per_cu) * cus / S);
  return teams >= 2 ? static_cast<int>(teams) : 0;
}

}  // namespace

int prep_int8_single_read(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                          const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                          const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                          int64_t T, int64_t H, int64_t D, int64_t block, uint16_t* kc,
                          uint16_t* vc, int64_t npad, float* qbar, float* kc_mean, float* kc_var,
                          float* vamax_part, float* vscale, int8_t* qi, float* qs, int8_t* ki,
                          float* ks, int ks_head_major, int8_t* vi, int64_t TP, uint32_t* sync,
                          int64_t sync_bytes, hipStream_t stream) {
  SOLATTN_REQUIRE(D == kHeadDim, SOLATTN_EUNSUPPORTED, "prep_int8: head_dim %lld != 128", (long long)D);
  SOLATTN_REQUIRE(block == 64 || block == 128, SOLATTN_EUNSUPPORTED,
                  "prep_int8: block %lld not in {64, 128}", (long long)block);
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && B * H < (1ll << 30) && T < (1ll << 31),
                  SOLATTN_EINVAL, "prep_int8: bad sizes");
  const int64_t NT = cdiv(T, block);
  SOLATTN_REQUIRE(npad >= NT && TP >= T, SOLATTN_EINVAL, "prep_int8: npad < NT or TP < T");
  const bool pv = vscale != nullptr;
  SOLATTN_REQUIRE(kc && vc && qbar && kc_mean && kc_var && qi && qs && ki && ks &&
                      (!pv || (vamax_part && vi)),
                  SOLATTN_EINVAL, "prep_int8: null output");
  SOLATTN_REQUIRE(sync && sync_bytes >= single_read_sync_words(B, H) * 4, SOLATTN_ESIZE,
                  "prep_int8: sync buffer %lld < %lld bytes", (long long)sync_bytes,
                  (long long)(single_read_sync_words(B, H) * 4));
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(kc) % 16 == 0 && reinterpret_cast<uintptr_t>(qi) % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(ki) % 8 == 0 &&
                      reinterpret_cast<uintptr_t>(vamax_part) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(vi) % 8 == 0,
                  SOLATTN_EINVAL, "prep_int8: misaligned outputs");
  if (int rc = check_bthd(q, sq_b, sq_t, sq_h, "prep_int8 q")) return rc;
  if (int rc = check_bthd(k, sk_b, sk_t, sk_h, "prep_int8 k")) return rc;
  if (int rc = check_bthd(v, sv_b, sv_t, sv_h, "prep_int8 v")) return rc;
  const size_t lds = static_cast<size_t>(NT) * 8 * sizeof(float);
  SOLATTN_REQUIRE(lds <= 64 * 1024, SOLATTN_EUNSUPPORTED,
                  "prep_int8: %lld blocks do not fit the single-read schedule", (long long)NT);
  const int nteams = single_read_teams(B, T, H, block, pv, lds);
  SOLATTN_REQUIRE(nteams > 0, SOLATTN_EUNSUPPORTED,
                  "prep_int8: B=%lld T=%lld H=%lld do not fit the single-read schedule on this "
                  "device (fewer than two heads' rows resident)",
                  (long long)B, (long long)T, (long long)H);
  PrepInt8Args a;
  a.q = q; a.k = k; a.v = v;
  a.sq_b = sq_b; a.sq_t = sq_t; a.sq_h = sq_h;
  a.sk_b = sk_b; a.sk_t = sk_t; a.sk_h = sk_h;
  a.sv_b = sv_b; a.sv_t = sv_t; a.sv_h = sv_h;
  a.T = T; a.TP = TP; a.npad = npad;
  a.B = static_cast<int>(B); a.H = static_cast<int>(H); a.NT = static_cast<int>(NT);
  a.S = static_cast<int>(cdiv(T, kSpan)); a.nteams = nteams;
  a.kc = kc; a.vc = vc; a.qbar = qbar; a.kc_mean = kc_mean; a.kc_var = kc_var;
  a.vscale = vscale; a.vamax_part = pv ? vamax_part : nullptr;
  a.qi = qi; a.ki = ki; a.vi = vi; a.qs = qs; a.ks = ks;
  a.ks_st = ks_head_major ? 1 : H;
  a.ks_sh = ks_head_major ? TP : 1;
  a.sync = sync;
  hipLaunchKernelGGL(sync_init_kernel, dim3(1), dim3(256), 0, stream, sync, nteams + 1);
  if (int rc = check_launch("prep_int8 sync init")) return rc;
  const void* kern = block == 64 ? (pv ? single_read_kernel<64, true>() : single_read_kernel<64, false>())
                                 : (pv ? single_read_kernel<128, true>() : single_read_kernel<128, false>());
  void* args[] = {&a};
  const hipError_t e = hipLaunchCooperativeKernel(kern, dim3(static_cast<uint32_t>(nteams) * a.S),
                                                  dim3(kPoolThreads), args, lds, stream);
  if (e != hipSuccess) {
    (void)hipGetLastError();
    return set_error(SOLATTN_ELAUNCH, "prep_int8: cooperative launch of %d x %d workgroups: %s",
                     nteams, a.S, hipGetErrorString(e));
  }
  return check_launch("prep_int8");
}

}  // namespace solattn

extern "C" int64_t solattn_prep_int8_sync_bytes(int64_t B, int64_t H) {
  if (B <= 0 || H <= 0) return 0;
  return cdiv(single_read_sync_words(B, H) * 4, 256) * 256;
}

extern "C" int solattn_prep_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                 const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                                 const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                 int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                                 uint16_t* kc, uint16_t* vc, int64_t npad, float* qbar,
                                 float* kc_mean, float* kc_var, float* vamax_part, float* vscale,
                                 int8_t* qi, float* qs, int8_t* ki, float* ks, int ks_head_major,
                                 int8_t* vi, int64_t TP, void* sync, int64_t sync_bytes,
                                 solattn_stream_t stream) {
  clear_error();
  return prep_int8_single_read(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B,
                               T, H, D, block, kc, vc, npad, qbar, kc_mean, kc_var, vamax_part,
                               vscale, qi, qs, ki, ks, ks_head_major, vi, TP,
                               static_cast<uint32_t*>(sync), sync_bytes,
                               reinterpret_cast<hipStream_t>(stream));
}
