// BF16 Sol-Attn forward on gfx950 MFMA.
//
// One workgroup per (batch, head, query block of BLK rows); each wave owns 32
// query rows. Work is a list of 64-key tiles in LDS (double buffered):
//   pooled tiles  64 pooled keys kc_j / values vc_j, masked to the approximate
//                 blocks of this query block, softmax weight x len_j
//                 (/root/reference/_tri_fwd.py:288-308);
//   exact tiles   64 tokens of an exact block (/root/reference/_tri_fwd.py:310-340).
// All tiles feed one online softmax per query row.
//
// MFMA dataflow (v_mfma_f32_32x32x16_bf16): S^T = K . Q^T puts one query row
// per lane column, so row max / sum need one cross-lane step (lane ^ 32) and
// the S accumulator converts in place into the B operand of O^T += V^T . P^T.
// Tiles are copied global -> LDS directly (no VGPR staging, so two waves fit
// per SIMD); V stays row-major and ds_read_tr16_b64 delivers it transposed as
// the MFMA A operand. XOR-swizzled chunks keep the LDS reads conflict free.
#include "common.hpp"
#include "fwd_common.hpp"

namespace solattn {

// Two MFMA steps (d = 32*cc0 .. 32*cc0 + 31) of S^T = K . Q^T into s; the
// first step starts from a zero accumulator (an inline constant operand).
template <bool FIRST>
__device__ __forceinline__ void qk_steps(const uint16_t* kt, const bf16x8 (&qreg)[8], int col,
                                         int half, f32x16 (&s)[2], int cc0) {
  const f32x16 zero = {};
#pragma unroll
  for (int cc = cc0; cc < cc0 + 2; ++cc)
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = 32 * m + col;
      const bf16x8 a =
          *reinterpret_cast<const bf16x8*>(&kt[row * kD + swz_k(row, 2 * cc + half) * 8]);
      s[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[cc], (FIRST && cc == cc0) ? zero : s[m],
                                                     0, 0, 0);
    }
}

// Keys outside the tile's mask get -inf. Lane (col, half) holds key
// 32m + 8i + 4*half + j in element 4i + j of s[m].
__device__ __forceinline__ void mask_scores(f32x16 (&s)[2], uint64_t amask, int half) {
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const uint32_t bits = static_cast<uint32_t>(amask >> (32 * m + 4 * half));
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
      for (int j = 0; j < 4; ++j)
        s[m][4 * i + j] = ((bits >> (8 * i + j)) & 1u) ? s[m][4 * i + j] : -INFINITY;
  }
}

// Row sum of a pooled tile: key j weighs len_j, i.e. BLK except the ragged
// last block (/root/reference/_tri_fwd.py:302-307).
template <int BLK>
__device__ __forceinline__ float pooled_sum(const f32x16 (&p)[2], int first, int half, int NT, int T) {
  const int kl_last = NT - 1 - first;
  const float tail = static_cast<float>(T - (NT - 1) * BLK);
  float sum = 0.f;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int kl = 32 * m + 8 * (r >> 2) + 4 * half + (r & 3);
      sum = fmaf(p[m][r], kl == kl_last ? tail : static_cast<float>(BLK), sum);
    }
  return sum;
}

__device__ __forceinline__ float max16(const f32x16& v, float mx) {
#pragma unroll
  for (int r = 0; r < 16; ++r) mx = fmaxf(mx, v[r]);
  return mx;
}

__device__ __forceinline__ float exp16(f32x16& v, float c, float neg) {
  float sum = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    v[r] = __builtin_amdgcn_exp2f(fmaf(v[r], c, neg));
    sum += v[r];
  }
  return sum;
}

// One pipelined step: the QK MFMAs of tile n+1 (into sn) are interleaved with
// the softmax of tile n (in sc), then P.V of tile n. On entry K(n+1) and V(n)
// are in LDS; this step starts the copies of K(n+2) and V(n+1) into the
// buffers freed by step n-1.
template <int BLK, int NTHREADS>
__device__ __forceinline__ void fwd_step(int n, int ntiles, f32x16 (&sc)[2], f32x16 (&sn)[2],
                                         SoftmaxState& st, uint16_t (*kbuf)[kTileElems],
                                         uint16_t (*vbuf)[kTileElems], const TileList& tl,
                                         const KVSource& src, const TileOffsets<NTHREADS>& off,
                                         const bf16x8 (&qreg)[8], int lane, float c, int T, int NT) {
  const int col = lane & 31, half = lane >> 5;
  if (n + 2 < ntiles) issue_half<BLK, NTHREADS>(kbuf[n & 1], 0, tl, n + 2, src, off, T, NT);
  if (n + 1 < ntiles) issue_half<BLK, NTHREADS>(vbuf[(n + 1) & 1], 1, tl, n + 1, src, off, T, NT);
  const TileDesc td = tile_desc<BLK>(tl, n, T, NT);
  const uint16_t* kt = kbuf[(n + 1) & 1];

  if (td.amask != ~0ull) mask_scores(sc, td.amask, half);

  qk_steps<true>(kt, qreg, col, half, sn, 0);
  float mx = max16(sc[0], -INFINITY);
  qk_steps<false>(kt, qreg, col, half, sn, 2);
  mx = max16(sc[1], mx);
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  // The running max moves only when the tile's max exceeds it by more than
  // kMaxSlack (log2 units), so the O rescale is rare.
  const float m_tile = mx * c;
  const float m_new = m_tile > st.m + kMaxSlack ? m_tile : st.m;
  const float alpha = st.m == m_new ? 1.f : __builtin_amdgcn_exp2f(st.m - m_new);
  const float neg = -m_new;
  qk_steps<false>(kt, qreg, col, half, sn, 4);
  float psum = exp16(sc[0], c, neg);
  qk_steps<false>(kt, qreg, col, half, sn, 6);
  psum += exp16(sc[1], c, neg);
  if (td.pooled) psum = pooled_sum<BLK>(sc, td.first, half, NT, T);
  st.l = fmaf(st.l, alpha, psum);
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[dt][r] *= alpha;
  }
  st.m = m_new;

  pv_tr16(vbuf[n & 1], sc, lane, st.acc);
  wait_tile_copies();
  __syncthreads();
}

template <int BLK>
__global__ void __launch_bounds__(BLK * 2, 2)
fwd_bf16_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t npad,
                const int32_t* __restrict__ counts, const int16_t* __restrict__ lists,
                const uint32_t* __restrict__ mask, int T, int H, int NT, int W, float c,
                uint16_t* __restrict__ o, int64_t so_b, int64_t so_t, int64_t so_h) {
  constexpr int NTHREADS = BLK * 2;
  __shared__ __align__(16) uint16_t kbuf[2][kTileElems];
  __shared__ __align__(16) uint16_t vbuf[2][kTileElems];
  __shared__ TileList tl;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  int bh, qb;
  tile_coords(blockIdx.x, gridDim.x, NT, bh, qb);
  const int b = bh / H, h = bh % H;
  const int64_t row = static_cast<int64_t>(bh) * NT + qb;

  const int ntiles = build_tile_list<BLK>(tl, counts, lists, mask, row, NT, W, T);
  if (ntiles == 0) return;  // cannot happen for routed lists: the diagonal is exact

  const KVSource src{k + b * sk_b + h * sk_h, sk_t, v + b * sv_b + h * sv_h, sv_t,
                     kc + (static_cast<int64_t>(b) * npad * H + h) * kD,
                     static_cast<int64_t>(H) * kD, vc + (static_cast<int64_t>(b) * npad * H + h) * kD};
  TileOffsets<NTHREADS> off;
  off.init(sk_t, sv_t);
  issue_half<BLK, NTHREADS>(kbuf[0], 0, tl, 0, src, off, T, NT);
  issue_half<BLK, NTHREADS>(vbuf[0], 1, tl, 0, src, off, T, NT);
  if (ntiles > 1) issue_half<BLK, NTHREADS>(kbuf[1], 0, tl, 1, src, off, T, NT);

  // This wave's 32 query rows as the B operand of S^T = K Q^T.
  const int qrow = qb * BLK + wave * 32 + col;
  bf16x8 qreg[8];
  {
    const uint16_t* qp = q + b * sq_b + static_cast<int64_t>(qrow) * sq_t + h * sq_h + half * 8;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      uint4 r = make_uint4(0u, 0u, 0u, 0u);
      if (qrow < T) r = *reinterpret_cast<const uint4*>(qp + cc * 16);
      qreg[cc] = __builtin_bit_cast(bf16x8, r);
    }
  }

  SoftmaxState st;
  st.init();
  wait_tile_copies();
  __syncthreads();
  f32x16 sa[2], sb[2];
  qk_swz(kbuf[0], qreg, col, half, sa);
  __syncthreads();  // kbuf[0] is refilled (K of tile 2) by the first step

  // Unrolled by two so the S buffers swap roles without register copies.
  for (int n = 0; n < ntiles; n += 2) {
    fwd_step<BLK, NTHREADS>(n, ntiles, sa, sb, st, kbuf, vbuf, tl, src, off, qreg, lane, c, T, NT);
    if (n + 1 < ntiles)
      fwd_step<BLK, NTHREADS>(n + 1, ntiles, sb, sa, st, kbuf, vbuf, tl, src, off, qreg, lane, c, T, NT);
  }

  store_output(st, o + b * so_b + h * so_h, so_t, qrow, T, half);
}

}  // namespace solattn

using namespace solattn;

extern "C" int solattn_fwd_bf16(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                                const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                const uint16_t* kc, const uint16_t* vc, int64_t npad,
                                const int32_t* counts, const int16_t* lists,
                                const uint32_t* mask, int64_t B, int64_t T, int64_t H, int64_t D,
                                int64_t block, float scale, uint16_t* o, int64_t so_b,
                                int64_t so_t, int64_t so_h, solattn_stream_t stream) {
  clear_error();
  if (int rc = check_fwd_args(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, kc,
                              vc, npad, counts, lists, mask, B, T, H, D, block, o, so_b, so_t,
                              so_h, "fwd_bf16"))
    return rc;
  const int64_t NT = cdiv(T, block);
  const int W = static_cast<int>(cdiv(NT, 32));
  const float c = scale * kLog2e;
  const uint32_t grid = static_cast<uint32_t>(B * H * NT);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (block == 128) {
    hipLaunchKernelGGL(fwd_bf16_kernel<128>, dim3(grid), dim3(256), 0, s,
                       q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, kc, vc, npad,
                       counts, lists, mask, static_cast<int>(T), static_cast<int>(H),
                       static_cast<int>(NT), W, c, o, so_b, so_t, so_h);
  } else {
    hipLaunchKernelGGL(fwd_bf16_kernel<64>, dim3(grid), dim3(128), 0, s, q,
                       sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, kc, vc, npad,
                       counts, lists, mask, static_cast<int>(T), static_cast<int>(H),
                       static_cast<int>(NT), W, c, o, so_b, so_t, so_h);
  }
  return check_launch("fwd_bf16");
}
