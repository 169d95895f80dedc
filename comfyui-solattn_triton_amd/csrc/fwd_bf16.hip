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
  __shared__ SwzBuf buf[2];
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
  issue_tile<BLK, NTHREADS>(buf[0], tl, 0, src, off, T, NT);

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

  for (int n = 0; n < ntiles; ++n) {
    // Tile n+1 streams into the other buffer while tile n is computed; that
    // buffer's last readers finished before the barrier that ended tile n-1.
    if (n + 1 < ntiles) issue_tile<BLK, NTHREADS>(buf[(n + 1) & 1], tl, n + 1, src, off, T, NT);
    const TileDesc td = tile_desc<BLK>(tl, n, T, NT);
    const SwzBuf& tb = buf[n & 1];

    f32x16 s[2];
    qk_swz(tb, qreg, col, half, s);
    softmax_update<BLK>(st, s, td, c, half, NT, T);
    pv_tr16(tb, s, lane, st.acc);

    wait_tile_copies();
    __syncthreads();
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
