// BF16 Sol-Attn forward on gfx950 MFMA.
//
// One workgroup per (batch, head, query block of BLK rows); each wave owns 32
// query rows, two waves share a SIMD. Work is a list of 64-key tiles staged in
// LDS by global -> LDS copies (no VGPR staging):
//   pooled tiles  64 pooled keys kc_j / values vc_j, masked to the approximate
//                 blocks of this query block, softmax weight x len_j
//                 (/root/reference/_tri_fwd.py:288-308);
//   exact tiles   64 tokens of an exact block (/root/reference/_tri_fwd.py:310-340).
// All tiles feed one online softmax per query row, which is exact under any
// tile order (up to fp32 rounding). The full exact tiles run through a
// software pipeline, the pooled tiles and the ragged last exact tile through a
// plain path:
//   block 128 (fwd_bf16_kernel): K and V double buffered, two workgroups per
//     CU; exact tiles first, three-stage step n = S(n+1) = K(n+1) Q^T, O +=
//     P(n-1) V(n-1) and the softmax of S(n) in one instruction stream;
//   block 64 (fwd_bf16_sbuf_kernel): K and V single buffered, four workgroups
//     per CU; plain tiles first, two-stage step n = S(n+1) with the softmax of
//     tile n interleaved, then O += P(n) V(n).
// Both pipelined steps are hand-ordered: inline-asm MFMAs and softmax exp
// pairs in a fixed interleave (fwd_common.hpp), which the compiler's own
// schedule did not give.
//
// MFMA dataflow (v_mfma_f32_32x32x16_bf16): S^T = K . Q^T puts one query row
// per lane column, so row max / sum need one cross-lane step (lanes 32 apart,
// v_permlane32_swap) and the S accumulator converts in place into the B
// operand of O^T += V^T . P^T. V stays row-major in LDS and ds_read_b64_tr_b16
// delivers it transposed as the MFMA A operand. XOR-swizzled 16-byte chunks
// keep the LDS reads conflict free (fwd_common.hpp).
#include "common.hpp"
#include "fwd_common.hpp"

namespace solattn {
namespace bf16fwd {

// Pipelined step over full exact tile n (scores in sc): S(n+1) from the K tile
// kn goes to sn, interleaved with the softmax of tile n; `mid` runs before
// P(n) . V(n).
// kl, vl: this lane's operand addresses (k_lane, v_lane) in K(n+1) and V(n).
// Hand-ordered as step3 below: each score MFMA is followed by the exps of
// one P word, the operands are read two MFMAs ahead, and the lazy tile max
// works the same way (also catching the first exact tile when no plain tile
// came before it: running max -inf, p = inf).
template <typename Mid>
__device__ __forceinline__ void fast_step(SoftmaxState& st, f32x16 (&sc)[2], f32x16 (&sn)[2],
                                          uint32_t kl, uint32_t vl, const bf16x8 (&q)[8],
                                          float c, int lane, Mid&& mid) {
  bf16x8 ka[3], va[3], pb[4];
  uint32_t pw[4][4];
  float psum = 0.f;
  const float neg = -st.m;
  ka[0] = k_op_x(kl, 0, 0);
  ka[1] = k_op_x(kl, 1, 0);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i + 2 < 16) {
      ka[(i + 2) % 3] = k_op_x(kl, (i + 2) & 1, (i + 2) >> 1);
      asm volatile("" ::: "memory");
    }
    if (i < 2)
      mfma_v0(sn[i & 1], ka[i % 3], q[i >> 1]);
    else
      mfma_v(sn[i & 1], ka[i % 3], q[i >> 1]);
    const int ks = i >> 2, w = i & 3;
    const int r = 8 * (ks & 1) + 2 * w;
    pw[ks][w] = exp_pair(sc[ks >> 1][r], sc[ks >> 1][r + 1], c, neg, psum);
  }
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    pb[ks] = __builtin_bit_cast(bf16x8, make_uint4(pw[ks][0], pw[ks][1], pw[ks][2], pw[ks][3]));
  float alpha = 1.f;
  if (__any(!(psum <= 255.f))) {  // (also catches inf / NaN)
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(sc[0][r], sc[1][r]));
    const float m_new = new_max(st.m, xhalf_max(mx) * c, alpha);
    if (__any(m_new != st.m)) {  // lanes whose max stays recompute the same P
      st.m = m_new;
      psum = 0.f;
      psum = exp8<0>(sc[0], c, -m_new, pb[0], psum);
      psum = exp8<8>(sc[0], c, -m_new, pb[1], psum);
      psum = exp8<0>(sc[1], c, -m_new, pb[2], psum);
      psum = exp8<8>(sc[1], c, -m_new, pb[3], psum);
      mfma_fence(st.acc);  // the rescale reads O
      rescale(st, alpha);
    }
  }
  st.l = fmaf(st.l, alpha, psum);
  mid();
  va[0] = v_op_x(vl, 0, 0);
  va[1] = v_op_x(vl, 0, 1);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i + 2 < 16) {
      va[(i + 2) % 3] = v_op_x(vl, (i + 2) >> 2, (i + 2) & 3);
      asm volatile("" ::: "memory");
    }
    if (i == 0)
      mfma_v_first(st.acc[0], va[0], pb[0]);
    else if (i == 15)
      mfma_v_tie(st.acc[3], va[0], pb[3], sn);  // va[15 % 3]
    else
      mfma_v(st.acc[i & 3], va[i % 3], pb[i >> 2]);
  }
}

// Three-stage step: S(n+1) = K(n+1) Q^T, O += P(n-1) V(n-1) and the softmax of
// S(n) -> P(n) share one instruction stream, so the softmax's VALU work
// overlaps 32 MFMAs instead of 16. O is rescaled to the new running max after
// the P(n-1) V(n-1) products; P(n) V(n) is left to the next step. QK = false
// drops the score product (last tile), PV = false the value product (first).
// The two key halves of S(n+1) accumulate alternately (MFMA i adds channel
// chunk i/2 to half i%2), so consecutive score MFMAs are independent (with the
// halves one after the other, each a chain of 8, the loop ran 1.3-2% slower).
// kl, vl: this lane's operand addresses (k_lane, v_lane) in K(n+1) and V(n-1).
// The step is one hand-ordered stream (fwd_common.hpp: mfma_v*, exp_pair):
// slot i (16 per step) issues the MFMA of score chunk i, the exps of P(n)
// word i (two scores of S(n)), then the MFMA of P.V operand i; the K and V
// operands of slot i + 2 are read at the top of slot i (the empty asm with a
// memory clobber keeps the reads there, so each has two slots to land).
// Measured on a stand-alone copy of the loop: 1346 against 1250 TFLOP/s, the
// compiler's order having issued the MFMAs four at a time with the softmax
// between the groups.
// Lazy tile max: the exps use the running max as it stands, and the tile's max
// is taken only when a lane's row sum exceeds 255. No sum above 255 means every
// p <= 255, i.e. every score is below the running max + log2(255.5) <
// kMaxSlack, so the tile would not have moved the max: the running max evolves
// as with the max taken every step. The first exact tile of a workgroup
// (running max -inf, p = inf) always takes that path.
template <bool QK, bool PV>
__device__ __forceinline__ void step3(SoftmaxState& st, const f32x16 (&sc)[2], f32x16 (&sn)[2],
                                      const bf16x8 (&pp)[4], bf16x8 (&pn)[4], uint32_t kl,
                                      uint32_t vl, const bf16x8 (&q)[8], float c) {
  static_assert(kMaxSlack >= 8.f, "the lazy test relies on 255 < 2^kMaxSlack");
  bf16x8 ka[3], va[3];
  uint32_t pw[4][4];
  float psum = 0.f;
  const float neg = -st.m;
  if constexpr (QK) {
    ka[0] = k_op_x(kl, 0, 0);
    ka[1] = k_op_x(kl, 1, 0);
  }
  if constexpr (PV) {
    va[0] = v_op_x(vl, 0, 0);
    va[1] = v_op_x(vl, 0, 1);
  }
  asm volatile("" ::: "memory");
  const auto unit = [&](int i) {
    const int ks = i >> 2, w = i & 3;
    const int r = 8 * (ks & 1) + 2 * w;
    pw[ks][w] = exp_pair(sc[ks >> 1][r], sc[ks >> 1][r + 1], c, neg, psum);
  };
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i + 2 < 16) {
      if constexpr (QK) ka[(i + 2) % 3] = k_op_x(kl, (i + 2) & 1, (i + 2) >> 1);
      if constexpr (PV) va[(i + 2) % 3] = v_op_x(vl, (i + 2) >> 2, (i + 2) & 3);
      asm volatile("" ::: "memory");
    }
    if constexpr (QK) {
      // the two key halves of S(n+1) alternate (consecutive MFMAs independent)
      if (i < 2)
        mfma_v0(sn[i & 1], ka[i % 3], q[i >> 1]);
      else
        mfma_v(sn[i & 1], ka[i % 3], q[i >> 1]);
      unit(i);
    }
    if constexpr (PV) {
      if (i == 0)
        mfma_v_first(st.acc[0], va[0], pp[0]);
      else if (QK && i == 15)
        mfma_v_tie(st.acc[3], va[0], pp[3], sn);  // va[15 % 3]
      else
        mfma_v(st.acc[i & 3], va[i % 3], pp[i >> 2]);
    }
    if constexpr (!QK) unit(i);
    // Raised wave priority for the rest of the step: the issue arbiter then
    // prefers a wave inside its MFMA stream over one at its copies / barrier
    // (about 1-2% at cfg 2).
    if (i == 0) __builtin_amdgcn_s_setprio(1);
  }
  __builtin_amdgcn_s_setprio(0);
  if constexpr (QK && !PV) mfma_fence(sn);
  if constexpr (!QK) mfma_fence(st.acc);  // the plain path's builtin MFMAs follow
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    pn[ks] = __builtin_bit_cast(bf16x8, make_uint4(pw[ks][0], pw[ks][1], pw[ks][2], pw[ks][3]));
  float alpha = 1.f;
  if (__any(!(psum <= 255.f))) {  // (also catches inf / NaN)
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(sc[0][r], sc[1][r]));
    const float m_new = new_max(st.m, xhalf_max(mx) * c, alpha);
    if (__any(m_new != st.m)) {  // lanes whose max stays recompute the same P
      st.m = m_new;
      psum = 0.f;
      psum = exp8<0>(sc[0], c, -m_new, pn[0], psum);
      psum = exp8<8>(sc[0], c, -m_new, pn[1], psum);
      psum = exp8<0>(sc[1], c, -m_new, pn[2], psum);
      psum = exp8<8>(sc[1], c, -m_new, pn[3], psum);
      if constexpr (PV) mfma_fence(st.acc);  // the rescale reads O
      rescale(st, alpha);
    }
  }
  st.l = fmaf(st.l, alpha, psum);
}

// Tile n of this kernel's order: pooled tiles, the ragged exact tile (if
// any), then the full exact tiles in ascending key order.
template <int BLK>
__device__ __forceinline__ TileDesc desc(const TileList& tl, int n, int nrag, int T, int NT) {
  if (n < tl.npool) return pooled_desc(tl, n, NT);
  if (n < tl.npool + nrag) return exact_desc<BLK>(tl, tl.nexact - 1, T, NT);
  return exact_desc<BLK>(tl, n - tl.npool - nrag, T, NT);
}

// Block 64 forward (workgroups of 2 waves). K and V are single buffered
// (32 KiB), so four workgroups and two waves per SIMD fit a CU; the pipeline
// step waits twice (K refilled after the QK phase, V after P.V). Tile order:
// pooled tiles, the ragged exact tile (if any), then the full exact tiles.
template <int BLK>
__global__ void __launch_bounds__(BLK * 2) __attribute__((amdgpu_waves_per_eu(2)))
fwd_bf16_sbuf_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t npad,
                const int32_t* __restrict__ counts, const uint32_t* __restrict__ mask, int T, int H, int NT, int W, float c,
                uint16_t* __restrict__ o, int64_t so_b, int64_t so_t, int64_t so_h) {
  constexpr int NTHREADS = BLK * 2;
  __shared__ __align__(256) uint16_t kbuf[kTileElems];
  __shared__ __align__(256) uint16_t vbuf[kTileElems];
  __shared__ TileList tl;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  int bh, qb;
  tile_coords_lpt<kLptTokens / BLK>(counts, NT, bh, qb);
  const int b = bh / H, h = bh % H;
  const int64_t row = static_cast<int64_t>(bh) * NT + qb;

  const int ntiles = build_tile_list<BLK>(tl, mask, row, NT, W, T);
  if (ntiles == 0) return;  // cannot happen for routed masks: the diagonal is exact
  // The last exact tile is ragged when block NT-1 is exact and T is not a
  // multiple of 64 (exact blocks are listed in ascending order).
  const int nrag = ragged_tiles(tl, NT, T);
  const int nplain = tl.npool + nrag;

  const KVSource src{k + b * sk_b + h * sk_h, sk_t, v + b * sv_b + h * sv_h, sv_t,
                     kc + (static_cast<int64_t>(b) * npad * H + h) * kD,
                     static_cast<int64_t>(H) * kD, vc + (static_cast<int64_t>(b) * npad * H + h) * kD};
  CopyOffsets<NTHREADS> off;
  off.init(sk_t, sv_t);
  const uint32_t kb = lds_addr(kbuf), vb = lds_addr(vbuf);  // LDS byte addresses
  const uint32_t kl = k_lane(kb, col, half), vl = v_lane(vb, lane);  // this lane's operands
  const auto first_of = [&](int n) { return exact_first<BLK>(tl, n - nplain); };
  const auto issue_k_at = [&](int first) {
    issue_full<NTHREADS>(kb, src.k + static_cast<int64_t>(first) * src.sk, src.sk, off.k);
  };
  const auto issue_v_at = [&](int first) {
    issue_full<NTHREADS>(vb, src.v + static_cast<int64_t>(first) * src.sv, src.sv, off.v);
  };
  const auto issue_k = [&](int n) { issue_k_at(first_of(n)); };
  const auto issue_v = [&](int n) { issue_v_at(first_of(n)); };
  const auto issue_tile = [&](int n) {
    if (n >= nplain) {
      issue_k(n);
      issue_v(n);
    } else {
      const TileDesc td = desc<BLK>(tl, n, nrag, T, NT);
      issue_generic<NTHREADS>(kb, 0, td, src);
      issue_generic<NTHREADS>(vb, 1, td, src);
    }
  };
  issue_tile(0);

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

  // ---- plain tiles (pooled, ragged). The next tile's K is copied once
  // every wave has its scores (it lands during the softmax and P.V), its V
  // once every wave is done with P.V (it lands during the next QK).
  const auto issue_tile_kv = [&](int n, int kv) {
    if (n >= nplain) {
      if (kv == 0) issue_k(n); else issue_v(n);
    } else {
      issue_generic<NTHREADS>(kv == 0 ? kb : vb, kv, desc<BLK>(tl, n, nrag, T, NT), src);
    }
  };
  for (int n = 0; n < nplain; ++n) {
    wait_vmcnt<CopyOffsets<NTHREADS>::U>();  // K(n); V(n) may be in flight
    __syncthreads();
    f32x16 s[2];
    qk_tile(kl, qreg, s);
    wait_tile_copies();  // V(n)
    __syncthreads();     // every wave is done with K(n)
    if (n + 1 < ntiles) issue_tile_kv(n + 1, 0);
    finish_tile<BLK>(st, s, vl, desc<BLK>(tl, n, nrag, T, NT), c, lane, NT, T);
    __syncthreads();     // every wave is done with V(n)
    if (n + 1 < ntiles) issue_tile_kv(n + 1, 1);
  }

  // ---- full exact tiles, pipelined; tile F was issued. K(n+2) past the last
  // tile is clamped to it: a redundant copy that nothing reads afterwards,
  // which keeps the loop free of branches.
  const int F = nplain;
  if (F < ntiles) {
    f32x16 sa[2], sb[2];
    int n = F;
    wait_tile_copies();
    __syncthreads();
    qk_tile(kl, qreg, sa);
    mfma_fence(sa);   // the step's softmax reads S(F) through asm
    __syncthreads();  // kbuf is free
    if (F + 1 < ntiles) issue_k(F + 1);
    wait_tile_copies();
    __syncthreads();  // K(F+1) and V(F) in LDS
    // Step n computes S(n+1) and needs n + 1 < ntiles. On entry kbuf holds
    // K(n+1), vbuf V(n) (copy possibly in flight). The first token rows of
    // the step's two copies were read from the LDS list in the step before
    // (kf, vf), so no copy waits on an LDS read.
    int kf = first_of(min(n + 2, ntiles - 1)), vf = first_of(n + 1);
    const auto step = [&](f32x16 (&sc)[2], f32x16 (&sn)[2]) {
      fast_step(st, sc, sn, kl, vl, qreg, c, lane, [&] {
        wait_tile_copies();  // V(n)
        __syncthreads();     // every wave is done with K(n+1)
        issue_k_at(kf);      // K(min(n + 2, ntiles - 1))
      });
      asm volatile("" ::: "memory");  // the list reads stay behind the MFMA stream
      const int kf_next = first_of(min(n + 3, ntiles - 1));
      const int vf_next = first_of(min(n + 2, ntiles - 1));
      wait_tile_copies();  // K(n+2)
      __syncthreads();     // every wave is done with V(n)
      issue_v_at(vf);      // V(n + 1)
      kf = kf_next;
      vf = vf_next;
      ++n;
    };
    // Pairs of steps, so the S buffers swap roles without register copies.
    while (n + 2 < ntiles) {
      step(sa, sb);
      step(sb, sa);
    }
    const TileDesc full{0, 0, kKeys, ~0ull};
    if (n + 1 < ntiles) {
      step(sa, sb);
      wait_tile_copies();
      __syncthreads();
      mfma_fence(st.acc);  // O from the asm MFMAs, read by the plain path
      finish_tile<BLK>(st, sb, vl, full, c, lane, NT, T);
    } else {
      wait_tile_copies();
      __syncthreads();
      mfma_fence(st.acc);
      finish_tile<BLK>(st, sa, vl, full, c, lane, NT, T);
    }
  }
  wait_tile_copies();

  store_rows(st, o + b * so_b + h * so_h, so_t, qrow, T, half);
}

// Block 128 forward with the three-stage pipeline. Tile order: the full
// exact tiles first (list tiles 0 .. nfast-1, ascending keys), then the
// ragged exact tile (if any) and the pooled tiles. K and V are double
// buffered (64 KiB, two workgroups per CU). The full exact phase runs first
// so that the plain phase's registers are not live across its loop.
template <int BLK>
__global__ void __launch_bounds__(BLK * 2) __attribute__((amdgpu_waves_per_eu(2)))
fwd_bf16_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                     const uint16_t* __restrict__ k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                     const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                     const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc, int64_t npad,
                     const int32_t* __restrict__ counts, const uint32_t* __restrict__ mask, int T, int H, int NT, int W, float c,
                     uint16_t* __restrict__ o, int64_t so_b, int64_t so_t, int64_t so_h) {
  constexpr int NTHREADS = BLK * 2;
  constexpr int kCopiesPerTile = 2 * CopyOffsets<NTHREADS>::U;
  __shared__ __align__(256) uint16_t kbuf[2][kTileElems];
  __shared__ __align__(256) uint16_t vbuf[2][kTileElems];
  __shared__ TileList tl;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  int bh, qb;
  tile_coords_lpt<kLptTokens / BLK>(counts, NT, bh, qb);
  const int b = bh / H, h = bh % H;
  const int64_t row = static_cast<int64_t>(bh) * NT + qb;

  const int ntiles = build_tile_list<BLK>(tl, mask, row, NT, W, T);
  if (ntiles == 0) return;  // cannot happen for routed masks: the diagonal is exact
  const int nrag = ragged_tiles(tl, NT, T);
  // Full exact tiles (list tiles 0 .. nfast-1) run through the pipeline when
  // there are at least two; a lone one runs as the first plain tile.
  const int nfast = ntiles - tl.npool - nrag;
  const int nlone = nfast == 1 ? 1 : 0;
  const int npipe = nfast - nlone;
  const int nplain = nlone + nrag + tl.npool;

  const KVSource src{k + b * sk_b + h * sk_h, sk_t, v + b * sv_b + h * sv_h, sv_t,
                     kc + (static_cast<int64_t>(b) * npad * H + h) * kD,
                     static_cast<int64_t>(H) * kD, vc + (static_cast<int64_t>(b) * npad * H + h) * kD};
  CopyOffsets<NTHREADS> off;
  off.init(sk_t, sv_t);
  const uint32_t kb = lds_addr(kbuf[0]), vb = lds_addr(vbuf[0]);  // LDS byte addresses
  const auto issue_k_at = [&](int first, int buf) {
    issue_full<NTHREADS>(kb + buf * kTileBytes, src.k + static_cast<int64_t>(first) * src.sk, src.sk, off.k);
  };
  const auto issue_v_at = [&](int first, int buf) {
    issue_full<NTHREADS>(vb + buf * kTileBytes, src.v + static_cast<int64_t>(first) * src.sv, src.sv, off.v);
  };
  const auto issue_k = [&](int e, int buf) { issue_k_at(exact_first<BLK>(tl, e), buf); };
  const auto issue_v = [&](int e, int buf) { issue_v_at(exact_first<BLK>(tl, e), buf); };
  // Plain tile p: the lone full exact tile (p < nlone), the ragged exact tile
  // (p < nlone + nrag), then the pooled tiles.
  const auto plain_desc = [&](int p) {
    if (p < nlone) return exact_desc<BLK>(tl, 0, T, NT);
    if (p < nlone + nrag) return exact_desc<BLK>(tl, tl.nexact - 1, T, NT);
    return pooled_desc(tl, p - nlone - nrag, NT);
  };
  const auto issue_plain_k = [&](int p, int buf) {
    issue_generic<NTHREADS>(kb + buf * kTileBytes, 0, plain_desc(p), src);
  };
  const auto issue_plain_v = [&](int p, int buf) {
    issue_generic<NTHREADS>(vb + buf * kTileBytes, 1, plain_desc(p), src);
  };
  if (npipe > 0) {
    issue_k(0, 0);
    issue_v(0, 0);
    issue_k(1, 1);
  } else {
    issue_plain_k(0, 0);
    issue_plain_v(0, 0);
  }

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
  int pbuf = 0;  // buffer of plain tile 0
  // This lane's operand addresses in K / V buffer 0 (buffer 1 is kTileBytes on).
  const uint32_t kl0 = k_lane(kb, col, half);
  const uint32_t vl0 = v_lane(vb, lane);

  // ---- full exact tiles. On entry to step n (0 < n < npipe): S(n) and
  // P(n-1) in registers, K(n+1) and V(n-1) in LDS; the step copies K(n+2)
  // over K(n) and V(n) over V(n-2). K(n+2) past the last tile is clamped to
  // it: a redundant copy into a buffer nothing reads afterwards.
  if (npipe > 0) {
    f32x16 sa[2], sb[2];
    wait_tile_copies();
    __syncthreads();
    qk_tile(kl0, qreg, sa);
    mfma_fence(sa);   // the step's softmax reads S(0) through asm
    __syncthreads();  // every wave is done with K(0)
    {
      const int E = npipe;
      bf16x8 pa[4], pb[4];
      issue_k(min(2, E - 1), 0);
      // First token rows of the tiles the next step copies, read from the LDS
      // list one step ahead: each step issues its copies from scalars it
      // already holds instead of waiting on an LDS read first.
      int kf = exact_first<BLK>(tl, min(3, E - 1)), vf = exact_first<BLK>(tl, 1);
      step3<true, false>(st, sa, sb, pb, pa, kl0 + kTileBytes, 0u, qreg, c);
      wait_tile_copies();
      __syncthreads();
      int n = 1;  // S(n) in sb, P(n-1) in pa
      const auto gstep = [&](const f32x16 (&sc)[2], f32x16 (&sn)[2], const bf16x8 (&pp)[4],
                             bf16x8 (&pn)[4]) {
        issue_k_at(kf, n & 1);  // K(min(n + 2, E - 1))
        issue_v_at(vf, n & 1);  // V(n)
        step3<true, true>(st, sc, sn, pp, pn, kl0 + ((n + 1) & 1) * kTileBytes,
                                vl0 + ((n - 1) & 1) * kTileBytes, qreg, c);
        // after the MFMA stream, so the read's latency overlaps the copy wait
        // and the barrier below rather than delaying this step's first MFMAs
        asm volatile("" ::: "memory");
        kf = exact_first<BLK>(tl, min(n + 3, E - 1));
        vf = exact_first<BLK>(tl, n + 1);
        wait_tile_copies();
        __syncthreads();
        ++n;
      };
      // Last tile n = E-1: no K left. Plain tile 0 is copied into the buffers
      // of tile n-1 while P(n-1) V(n-1), the softmax of S(n) and P(n) V(n) run.
      const auto last = [&](const f32x16 (&sc)[2], f32x16 (&dummy)[2], const bf16x8 (&pp)[4],
                            bf16x8 (&pn)[4]) {
        pbuf = (n - 1) & 1;
        issue_v_at(vf, n & 1);  // V(n)
        if (nplain > 0) issue_plain_k(0, pbuf);
        step3<false, true>(st, sc, dummy, pp, pn, 0u, vl0 + pbuf * kTileBytes, qreg, c);
        if (nplain > 0)
          wait_vmcnt<kCopiesPerTile / 2>();  // V(n) landed; plain K(0) may be in flight
        else
          wait_tile_copies();
        __syncthreads();  // every wave is done with V(n-1)
        if (nplain > 0) issue_plain_v(0, pbuf);
        pv_tile(vl0 + (n & 1) * kTileBytes, pn, lane, st.acc);
      };
      // Pairs of steps, so the S and P buffers swap roles without copies.
      while (n + 2 < E) {
        gstep(sb, sa, pa, pb);
        gstep(sa, sb, pb, pa);
      }
      if (n + 1 < E) {
        gstep(sb, sa, pa, pb);
        last(sa, sb, pb, pa);
      } else {
        last(sb, sa, pa, pb);
      }
      __syncthreads();  // every wave is done with V(E-1) before plain tile 1 lands there
    }
  }

  // ---- ragged and pooled tiles; plain tile p sits in buffers (pbuf + p) & 1
  for (int p = 0; p < nplain; ++p) {
    const int cur = (pbuf + p) & 1;
    if (p + 1 < nplain) {
      issue_plain_k(p + 1, cur ^ 1);
      issue_plain_v(p + 1, cur ^ 1);
      wait_vmcnt<kCopiesPerTile>();  // tile p landed; tile p+1 stays in flight
    } else {
      wait_tile_copies();
    }
    __syncthreads();
    f32x16 s[2];
    qk_tile(kl0 + cur * kTileBytes, qreg, s);
    finish_tile<BLK>(st, s, vl0 + cur * kTileBytes, plain_desc(p), c, lane, NT, T);
    __syncthreads();
  }
  wait_tile_copies();

  store_rows(st, o + b * so_b + h * so_h, so_t, qrow, T, half);
}

}  // namespace bf16fwd
}  // namespace solattn

using namespace solattn;

extern "C" int solattn_fwd_bf16(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                                const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                const uint16_t* kc, const uint16_t* vc, int64_t npad,
                                const int32_t* counts, const uint32_t* mask, int64_t B, int64_t T, int64_t H, int64_t D,
                                int64_t block, float scale, uint16_t* o, int64_t so_b,
                                int64_t so_t, int64_t so_h, solattn_stream_t stream) {
  clear_error();
  if (int rc = check_fwd_args(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, kc,
                              vc, npad, counts, mask, B, T, H, D, block, o, so_b, so_t,
                              so_h, "fwd_bf16"))
    return rc;
  const int64_t NT = cdiv(T, block);
  const int W = static_cast<int>(cdiv(NT, 32));
  const float c = scale * kLog2e;
  const uint32_t grid = static_cast<uint32_t>(B * H * NT);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (block == 128) {
    hipLaunchKernelGGL((bf16fwd::fwd_bf16_kernel<128>), dim3(grid), dim3(256), blist_lds_bytes(NT), s,
                       q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, kc, vc, npad,
                       counts, mask, static_cast<int>(T), static_cast<int>(H),
                       static_cast<int>(NT), W, c, o, so_b, so_t, so_h);
  } else {
    hipLaunchKernelGGL((bf16fwd::fwd_bf16_sbuf_kernel<64>), dim3(grid), dim3(128), blist_lds_bytes(NT), s, q,
                       sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, kc, vc, npad,
                       counts, mask, static_cast<int>(T), static_cast<int>(H),
                       static_cast<int>(NT), W, c, o, so_b, so_t, so_h);
  }
  return check_launch("fwd_bf16");
}
