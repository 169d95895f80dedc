// Pooling, moments, thresholds and routing for Sol-Attn on gfx950.
//
// Built with -ffp-contract=off: every fp32 operation below is rounded exactly
// where it is written, so the CPU oracle (oracle/solattn_oracle.c) reproduces
// kc, vc, qbar, thresholds and routing lists bit for bit.
//
//  pool    one pass over q, k, v per (block, head): 3 waves, one per tensor,
//          each lane holding 8 channels of one row in 16-byte loads; HBM-bound.
//  moments per-head kc mean / variance over blocks (+ INT8 centring, V scale).
//  route   thresholds, scores R[i][j] and per-query-block exact lists / masks.
#include <algorithm>

#include "common.hpp"

namespace solattn {

constexpr int kHeadDim = 128;

// ------------------------------------------------------------------ pool --
// /root/reference/_preprocess.py:23-113 (kc = sum/len, vc = sum, |v| max) and
// the q centroid of :140-149. Rows r of a block are split over 4 lane groups
// (r % 4 == lane / 16), each summing its rows in ascending order; the partials
// are combined (p0 + p1) + (p2 + p3) with two xor shuffles.
template <int BLK>
__global__ void __launch_bounds__(192)
pool_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
            const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
            const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t T,
            int H, int NT, uint16_t* __restrict__ kc, uint16_t* __restrict__ vc, int64_t npad,
            float* __restrict__ qbar, float* __restrict__ vamax_part) {
  const int j = blockIdx.x, h = blockIdx.y, b = blockIdx.z;
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const int g = lane >> 4;
  const int c8 = (lane & 15) * 8;
  const uint16_t* base;
  int64_t st;
  if (wave == 0) {
    base = k + b * sk_b + h * sk_h + c8;
    st = sk_t;
  } else if (wave == 1) {
    base = v + b * sv_b + h * sv_h + c8;
    st = sv_t;
  } else {
    base = q + b * sq_b + h * sq_h + c8;
    st = sq_t;
  }
  const int64_t t0 = static_cast<int64_t>(j) * BLK;
  float p[8], am[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) p[e] = am[e] = 0.f;
#pragma unroll 8
  for (int it = 0; it < BLK / 4; ++it) {
    const int64_t t = t0 + it * 4 + g;
    uint4 raw = make_uint4(0u, 0u, 0u, 0u);
    if (t < T) raw = *reinterpret_cast<const uint4*>(base + t * st);
    const uint32_t w[4] = {raw.x, raw.y, raw.z, raw.w};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float lo = lo_bf16(w[e]), hi = hi_bf16(w[e]);
      p[2 * e] = p[2 * e] + lo;
      p[2 * e + 1] = p[2 * e + 1] + hi;
      am[2 * e] = fmaxf(am[2 * e], fabsf(lo));
      am[2 * e + 1] = fmaxf(am[2 * e + 1], fabsf(hi));
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    p[e] = p[e] + __shfl_xor(p[e], 16);
    p[e] = p[e] + __shfl_xor(p[e], 32);
    am[e] = fmaxf(am[e], __shfl_xor(am[e], 16));
    am[e] = fmaxf(am[e], __shfl_xor(am[e], 32));
  }
  if (g != 0) return;
  const float flen = static_cast<float>(min<int64_t>(BLK, T - t0));
  const int64_t kv_off = ((b * npad + j) * H + h) * kHeadDim + c8;
  if (wave == 0) {
    uint4 o;
    o.x = pack_bf16x2(p[0] / flen, p[1] / flen);
    o.y = pack_bf16x2(p[2] / flen, p[3] / flen);
    o.z = pack_bf16x2(p[4] / flen, p[5] / flen);
    o.w = pack_bf16x2(p[6] / flen, p[7] / flen);
    *reinterpret_cast<uint4*>(kc + kv_off) = o;
  } else if (wave == 1) {
    uint4 o;
    o.x = pack_bf16x2(p[0], p[1]);
    o.y = pack_bf16x2(p[2], p[3]);
    o.z = pack_bf16x2(p[4], p[5]);
    o.w = pack_bf16x2(p[6], p[7]);
    *reinterpret_cast<uint4*>(vc + kv_off) = o;
    if (vamax_part) {
      float4* dst = reinterpret_cast<float4*>(
          vamax_part + ((static_cast<int64_t>(b) * NT + j) * H + h) * kHeadDim + c8);
      dst[0] = make_float4(am[0], am[1], am[2], am[3]);
      dst[1] = make_float4(am[4], am[5], am[6], am[7]);
    }
  } else {
    float4* dst = reinterpret_cast<float4*>(
        qbar + ((static_cast<int64_t>(b) * H + h) * NT + j) * kHeadDim + c8);
    dst[0] = make_float4(p[0] / flen, p[1] / flen, p[2] / flen, p[3] / flen);
    dst[1] = make_float4(p[4] / flen, p[5] / flen, p[6] / flen, p[7] / flen);
  }
}

// --------------------------------------------------------------- moments --
// /root/reference/_preprocess.py:241-243 and /root/reference/_fused_prep.py:77-81.
// 8 partial groups sum blocks j = g (mod 8) in ascending order; the partials
// are combined ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)).
__device__ __forceinline__ float tree8(const float (*part)[kHeadDim], int d) {
  return ((part[0][d] + part[1][d]) + (part[2][d] + part[3][d])) +
         ((part[4][d] + part[5][d]) + (part[6][d] + part[7][d]));
}

// One workgroup of 128 threads per (head, batch): thread t owns partial group
// g = t / 16 and channels c8 .. c8+7 (16-byte loads of 8 bf16). Loads are
// issued in chunks of kMomU before they are summed, in the same ascending
// order as a plain loop.
constexpr int kMomThreads = 128;
constexpr int kMomU = 16;
__device__ __forceinline__ void unpack8(const uint4& w, float (&x)[8]) {
  x[0] = lo_bf16(w.x); x[1] = hi_bf16(w.x); x[2] = lo_bf16(w.y); x[3] = hi_bf16(w.y);
  x[4] = lo_bf16(w.z); x[5] = hi_bf16(w.z); x[6] = lo_bf16(w.w); x[7] = hi_bf16(w.w);
}

__global__ void __launch_bounds__(kMomThreads)
moments_kernel(uint16_t* __restrict__ kc, int64_t npad, int NT, int H, int centre,
               float* __restrict__ kc_mean, float* __restrict__ kc_var,
               const float* __restrict__ vamax_part, float* __restrict__ vscale) {
  const int h = blockIdx.x, b = blockIdx.y;
  const int g = threadIdx.x >> 4, c8 = (threadIdx.x & 15) * 8;
  __shared__ float part[8][kHeadDim];
  __shared__ float amx[8][kHeadDim];
  __shared__ float smean[kHeadDim];
  const float fnt = static_cast<float>(NT);
  uint16_t* col = kc + (static_cast<int64_t>(b) * npad * H + h) * kHeadDim + c8;
  const int64_t sj = static_cast<int64_t>(H) * kHeadDim;
  float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float am[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j0 = g; j0 < NT; j0 += 8 * kMomU) {
    uint4 w[kMomU];
#pragma unroll
    for (int u = 0; u < kMomU; ++u)  // clamped row: no branch around the load
      w[u] = *reinterpret_cast<const uint4*>(col + min(j0 + 8 * u, NT - 1) * sj);
#pragma unroll
    for (int u = 0; u < kMomU; ++u) {
      if (j0 + 8 * u < NT) {
        float x[8];
        unpack8(w[u], x);
#pragma unroll
        for (int e = 0; e < 8; ++e) s[e] = s[e] + x[e];
      }
    }
  }
  if (vamax_part) {
    const float* a = vamax_part + (static_cast<int64_t>(b) * NT * H + h) * kHeadDim + c8;
    for (int j0 = g; j0 < NT; j0 += 8 * kMomU) {
      float4 w[kMomU][2];
#pragma unroll
      for (int u = 0; u < kMomU; ++u) {
        const float4* p = reinterpret_cast<const float4*>(a + min(j0 + 8 * u, NT - 1) * sj);
        w[u][0] = p[0];
        w[u][1] = p[1];
      }
#pragma unroll
      for (int u = 0; u < kMomU; ++u) {  // duplicated rows leave the max unchanged
        am[0] = fmaxf(am[0], w[u][0].x); am[1] = fmaxf(am[1], w[u][0].y);
        am[2] = fmaxf(am[2], w[u][0].z); am[3] = fmaxf(am[3], w[u][0].w);
        am[4] = fmaxf(am[4], w[u][1].x); am[5] = fmaxf(am[5], w[u][1].y);
        am[6] = fmaxf(am[6], w[u][1].z); am[7] = fmaxf(am[7], w[u][1].w);
      }
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    part[g][c8 + e] = s[e];
    amx[g][c8 + e] = am[e];
  }
  __syncthreads();
  {
    const int d = threadIdx.x;  // one channel per thread
    const float mean = tree8(part, d) / fnt;
    smean[d] = mean;
    kc_mean[(static_cast<int64_t>(b) * H + h) * kHeadDim + d] = mean;
    if (vamax_part) {
      float m = amx[0][d];
      for (int i = 1; i < 8; ++i) m = fmaxf(m, amx[i][d]);
      // absmax.div(127.0) in torch is a multiply by the fp32 reciprocal
      // (/root/reference/_fused_quant.py:104).
      const float sc = m * (1.0f / 127.0f);
      vscale[(static_cast<int64_t>(b) * H + h) * kHeadDim + d] = sc < 1e-8f ? 1e-8f : sc;
    }
  }
  __syncthreads();
  float mean[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) mean[e] = smean[c8 + e];
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  for (int j0 = g; j0 < NT; j0 += 8 * kMomU) {
    uint4 w[kMomU];
#pragma unroll
    for (int u = 0; u < kMomU; ++u)
      w[u] = *reinterpret_cast<const uint4*>(col + min(j0 + 8 * u, NT - 1) * sj);
#pragma unroll
    for (int u = 0; u < kMomU; ++u) {
      const int j = j0 + 8 * u;
      if (j < NT) {
        float x[8];
        unpack8(w[u], x);
        uint16_t nb[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          float y = x[e] - mean[e];
          if (centre) {
            nb[e] = f2bf(y);
            y = bf2f(nb[e]);
          }
          acc[e] = acc[e] + y * y;
        }
        if (centre) {
          uint4 o;
          o.x = nb[0] | (static_cast<uint32_t>(nb[1]) << 16);
          o.y = nb[2] | (static_cast<uint32_t>(nb[3]) << 16);
          o.z = nb[4] | (static_cast<uint32_t>(nb[5]) << 16);
          o.w = nb[6] | (static_cast<uint32_t>(nb[7]) << 16);
          *reinterpret_cast<uint4*>(col + j * sj) = o;
        }
      }
    }
  }
  __syncthreads();  // every thread has read part[] above
#pragma unroll
  for (int e = 0; e < 8; ++e) part[g][c8 + e] = acc[e];
  __syncthreads();
  {
    const int d = threadIdx.x;
    kc_var[(static_cast<int64_t>(b) * H + h) * kHeadDim + d] = tree8(part, d) / fnt;
  }
}

// ----------------------------------------------------------------- route --
// Thresholds (/root/reference/_preprocess.py:149-163, /root/reference/_fused_prep.py:50-59)
// and the routing rule of the forward (/root/reference/_tri_fwd.py:279-286),
// for kQB query blocks per workgroup; thread t scores key block j0 + t.
constexpr int kQB = 8;
constexpr int kRouteThreads = 256;
constexpr int kMaxWords = 512;  // NT <= 16384 (the forwards' limit)
constexpr int kKcStride = kHeadDim + 4;  // bf16 per staged kc row (264 B): conflict-free 8-byte reads
constexpr int kKcLoads = kHeadDim / 8;   // 16-byte loads per thread to stage 256 kc rows

__global__ void __launch_bounds__(kRouteThreads)
route_kernel(const float* __restrict__ qbar, const uint16_t* __restrict__ kc, int64_t npad,
             const float* __restrict__ kc_mean, const float* __restrict__ kc_var, int H, int NT,
             int W, float c, float c2, float tau, int mode, int64_t skv_lo, int64_t skv_hi,
             int64_t sq_lo, int64_t sq_hi, float* __restrict__ thr_out,
             int32_t* __restrict__ counts, int16_t* __restrict__ lists,
             uint32_t* __restrict__ mask) {
  const int i0 = blockIdx.x * kQB, h = blockIdx.y, b = blockIdx.z;
  const int t = threadIdx.x, wave = t >> 6, lane = t & 63;
  __shared__ __align__(16) float sq[kQB][kHeadDim];
  __shared__ float smk[kHeadDim], svk[kHeadDim];
  __shared__ float sthr[kQB];
  // exact bits of the kQB query blocks, W words each, in dynamic LDS
  extern __shared__ __align__(16) uint32_t smask_lds[];
  const auto smask = [&](int i, int w) -> uint32_t& { return smask_lds[i * W + w]; };
  __shared__ __align__(16) uint16_t skc[kRouteThreads * kKcStride];
  const int64_t bh = static_cast<int64_t>(b) * H + h;
  // The prologue's global loads are all issued before any of them is used:
  // the query centroids (one float4 per thread) and the moments.
  {
    static_assert(kQB * kHeadDim == 4 * kRouteThreads, "one float4 of qbar per thread");
    const int i = t / (kHeadDim / 4), d4 = t % (kHeadDim / 4);
    float4 qv = make_float4(0.f, 0.f, 0.f, 0.f);
    if (i0 + i < NT) qv = *reinterpret_cast<const float4*>(qbar + (bh * NT + i0 + i) * kHeadDim + 4 * d4);
    float mk = 0.f, vk = 0.f;
    if (t < kHeadDim) {
      mk = kc_mean[bh * kHeadDim + t];
      vk = kc_var[bh * kHeadDim + t];
    }
    *reinterpret_cast<float4*>(&sq[i][4 * d4]) = qv;
    if (t < kHeadDim) {
      smk[t] = mk;
      svk[t] = vk;
    }
  }
  for (int e = t; e < kQB * W; e += kRouteThreads) smask_lds[e] = 0u;
  __syncthreads();
  if (t < kQB) {
    float mu = 0.f, var = 0.f;
    for (int d = 0; d < kHeadDim; ++d) {
      const float qd = sq[t][d];
      if (mode == 0) mu = fmaf(qd, smk[d], mu);
      var = fmaf(qd * qd, svk[d], var);
    }
    float th;
    if (mode == 0) {
      mu = mu * c;
      var = var * c2;
      const float sd = sqrtf(fmaxf(var, 0.f) + 1e-6f);
      th = mu + tau * sd;
    } else {
      var = var * c2;
      th = tau * sqrtf(var + 1e-6f);
    }
    sthr[t] = th;
    if (i0 + t < NT) thr_out[(static_cast<int64_t>(b) * NT + i0 + t) * H + h] = th;
  }
  __syncthreads();

  for (int j0 = 0; j0 < NT; j0 += kRouteThreads) {
    // Stage kc rows j0 .. j0+255 (coalesced 16-byte loads, all issued before
    // the LDS stores; rows past NT are 0), then thread t scores row t.
    {
      uint4 v[kKcLoads];
#pragma unroll
      for (int u = 0; u < kKcLoads; ++u) {
        const int e = t + kRouteThreads * u;
        const int r = e >> 4, cc = e & 15;
        const int j = j0 + r;
        v[u] = make_uint4(0u, 0u, 0u, 0u);
        if (j < NT)
          v[u] = *reinterpret_cast<const uint4*>(
              kc + ((static_cast<int64_t>(b) * npad + j) * H + h) * kHeadDim + cc * 8);
      }
      __syncthreads();  // the previous chunk's rows have been read
#pragma unroll
      for (int u = 0; u < kKcLoads; ++u) {
        const int e = t + kRouteThreads * u;
        const int r = e >> 4, cc = e & 15;
        uint2* dst = reinterpret_cast<uint2*>(&skc[r * kKcStride + cc * 8]);
        dst[0] = make_uint2(v[u].x, v[u].y);
        dst[1] = make_uint2(v[u].z, v[u].w);
      }
    }
    __syncthreads();
    const int j = j0 + t;
    const bool active = j < NT;
    float acc[kQB];
#pragma unroll
    for (int i = 0; i < kQB; ++i) acc[i] = 0.f;
    const uint16_t* krow = &skc[t * kKcStride];
#pragma unroll 2
    for (int d4 = 0; d4 < kHeadDim / 4; ++d4) {
      const uint2 kw = *reinterpret_cast<const uint2*>(krow + 4 * d4);
      const float k0 = lo_bf16(kw.x), k1 = hi_bf16(kw.x);
      const float k2 = lo_bf16(kw.y), k3 = hi_bf16(kw.y);
#pragma unroll
      for (int i = 0; i < kQB; ++i) {
        const float4 qv = *reinterpret_cast<const float4*>(&sq[i][4 * d4]);
        acc[i] = fmaf(qv.x, k0, acc[i]);
        acc[i] = fmaf(qv.y, k1, acc[i]);
        acc[i] = fmaf(qv.z, k2, acc[i]);
        acc[i] = fmaf(qv.w, k3, acc[i]);
      }
    }
    const bool in_skv = j >= skv_lo && j < skv_hi;
#pragma unroll
    for (int i = 0; i < kQB; ++i) {
      const int qi = i0 + i;
      const float r = acc[i] * c;
      const int dij = qi > j ? qi - j : j - qi;
      const bool q_in_sink = qi >= sq_lo && qi < sq_hi;
      const bool routed = (r > sthr[i]) || dij <= 1 || in_skv;
      const bool exact = active && qi < NT && (q_in_sink || routed);
      const uint64_t bal = __ballot(exact);
      const int w0 = (j0 + wave * 64) >> 5;
      if (lane == 0 && w0 < W) {
        smask(i, w0) = static_cast<uint32_t>(bal);
        if (w0 + 1 < W) smask(i, w0 + 1) = static_cast<uint32_t>(bal >> 32);
      }
    }
  }
  __syncthreads();

  // Masks and ascending lists, one query block per wave at a time.
  for (int i = wave; i < kQB; i += kRouteThreads / 64) {
    const int qi = i0 + i;
    if (qi >= NT) break;
    const int64_t row = bh * NT + qi;
    int base = 0;
    for (int w0 = 0; w0 < W; w0 += 64) {
      const int w = w0 + lane;
      const uint32_t word = w < W ? smask(i, w) : 0u;
      if (w < W) mask[row * W + w] = word;
      const int cnt = __popc(word);
      int incl = cnt;
#pragma unroll
      for (int s = 1; s < 64; s <<= 1) {
        const int y = __shfl_up(incl, s);
        if (lane >= s) incl += y;
      }
      int off = base + incl - cnt;
      uint32_t bits = word;
      while (bits) {
        const int bit = __ffs(bits) - 1;
        bits &= bits - 1;
        lists[row * NT + off++] = static_cast<int16_t>(w * 32 + bit);
      }
      base += __shfl(incl, 63);
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

extern "C" int solattn_pool(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                            const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                            const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                            int64_t T, int64_t H, int64_t D, int64_t block, uint16_t* kc,
                            uint16_t* vc, int64_t npad, float* qbar, float* vamax_part,
                            solattn_stream_t stream) {
  clear_error();
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
  dim3 grid(static_cast<uint32_t>(NT), static_cast<uint32_t>(H), static_cast<uint32_t>(B));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (block == 64)
    hipLaunchKernelGGL(pool_kernel<64>, grid, dim3(192), 0, s, q, sq_b, sq_t, sq_h, k, sk_b, sk_t,
                       sk_h, v, sv_b, sv_t, sv_h, T, static_cast<int>(H), static_cast<int>(NT), kc,
                       vc, npad, qbar, vamax_part);
  else
    hipLaunchKernelGGL(pool_kernel<128>, grid, dim3(192), 0, s, q, sq_b, sq_t, sq_h, k, sk_b, sk_t,
                       sk_h, v, sv_b, sv_t, sv_h, T, static_cast<int>(H), static_cast<int>(NT), kc,
                       vc, npad, qbar, vamax_part);
  return check_launch("pool");
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
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(kc) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(vamax_part) % 16 == 0,
                  SOLATTN_EINVAL, "moments: kc and vamax_part must be 16-byte aligned");
  hipLaunchKernelGGL(moments_kernel, dim3(static_cast<uint32_t>(H), static_cast<uint32_t>(B)),
                     dim3(kMomThreads), 0, reinterpret_cast<hipStream_t>(stream), kc, npad,
                     static_cast<int>(NT), static_cast<int>(H), centre ? 1 : 0, kc_mean, kc_var,
                     vamax_part, vscale);
  return check_launch("moments");
}

extern "C" int solattn_route(const float* qbar, const uint16_t* kc, int64_t npad,
                             const float* kc_mean, const float* kc_var, int64_t B, int64_t T,
                             int64_t H, int64_t D, int64_t block, float scale, float tau, int mode,
                             int64_t sink_kv_lo, int64_t sink_kv_hi, int64_t sink_q_lo,
                             int64_t sink_q_hi, float* thr, int32_t* counts, int16_t* lists,
                             uint32_t* mask, solattn_stream_t stream) {
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
  SOLATTN_REQUIRE(qbar && kc && kc_var && (mode == 1 || kc_mean) && thr && counts && lists && mask,
                  SOLATTN_EINVAL, "route: null pointer");
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(kc) % 16 == 0, SOLATTN_EINVAL,
                  "route: kc must be 16-byte aligned");
  const float c = scale * kLog2e;
  const float c2 = c * c;
  dim3 grid(static_cast<uint32_t>(cdiv(NT, kQB)), static_cast<uint32_t>(H),
            static_cast<uint32_t>(B));
  hipLaunchKernelGGL(route_kernel, grid, dim3(kRouteThreads),
                     static_cast<size_t>(kQB * W * sizeof(uint32_t)),
                     reinterpret_cast<hipStream_t>(stream), qbar, kc, npad,
                     mode == 0 ? kc_mean : kc_var, kc_var, static_cast<int>(H),
                     static_cast<int>(NT), static_cast<int>(W), c, c2, tau, mode, sink_kv_lo,
                     sink_kv_hi, sink_q_lo, sink_q_hi, thr, counts, lists, mask);
  return check_launch("route");
}
