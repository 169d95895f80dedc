// INT8 Sol-Attn forward on gfx950 MFMA (/root/reference/_int8_fwd.py:208-372).
//
// Exact tiles: S = int32(qi . ki) * (qs*c * ks) on v_mfma_i32_32x32x32_i8.
//   INT8_PV: P is quantised per row against the max of its routed block,
//     pe = exp2(s - bmax), code = round(pe * 127), and multiplied with
//     per-channel int8 V on the i8 MFMA; the row factor beta/127 (beta =
//     exp2(bmax - m)) is applied per block, the channel scale vscale[d] once
//     after the exact blocks (it is the same for every block). Block 64: the
//     block is one 64-key tile (fwd_int8_kernel). Block 128:
//     fwd_int8_b128_kernel works on whole 128-key blocks; the tiles of a
//     ragged last block are quantised per 64-key tile.
//   otherwise: P.V in bf16 against the bf16 V, as in the BF16 forward.
// Pooled tiles run last in bf16 on the centred kc and vc. The online softmax
// is exact under any tile order, up to fp32 rounding.
//
// Tile order: the ragged exact tile (if any) through a plain path, the full
// exact tiles through a pipeline (step n: copies of K(n+2) and V(n+1); the i8
// MFMAs of S(n+1) interleaved with the softmax of tile n; P(n).V(n), then the
// conversion of S(n+1) to fp32 scores while tile n+1's ks are in LDS), then
// the pooled tiles. Tiles are copied global -> LDS directly: int8 K and V rows
// of 128 bytes with XOR-swizzled 16-byte chunks, ks behind the K rows;
// ds_read_b64_tr_b8 delivers int8 V transposed as the MFMA A operand.
#include "common.hpp"
#include "fwd_common.hpp"

namespace solattn {
namespace int8fwd {

constexpr int kI8Row = kD;                  // bytes per int8 K / V row
constexpr int kKsOffset = kKeys * kI8Row;   // ks[64] after the int8 K rows (bytes)

// 16 lanes per cycle read one 16-byte chunk of 16 consecutive rows; two 128-byte
// rows share a bank sweep, so rows of equal parity need distinct chunks.
__device__ __forceinline__ int swz_ki(int row, int chunk) { return chunk ^ ((row >> 1) & 7); }
// A ds_read_tr8 serves 32 lanes = 8 rows {0-3, 8-11} (+4 for the upper half)
// x 32 bytes; rows of equal parity get distinct chunk pairs.
__device__ __forceinline__ int swz_vi(int row, int chunk) {
  return chunk ^ (2 * (((row >> 1) & 1) | (((row >> 3) & 1) << 1)));
}

__device__ __forceinline__ i32x16 mfma_i8(const i32x4& a, const i32x4& b, const i32x16& c) {
  return __builtin_amdgcn_mfma_i32_32x32x32_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ i32x2 tr8(const char* p) {
  typedef int v2i32 __attribute__((ext_vector_type(2)));
  const v2i32 r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i32*)(p));
  return __builtin_bit_cast(i32x2, r);
}

// int8 K operand: key 32m + col, dims 32cc + 16half .. +15.
__device__ __forceinline__ i32x4 ki_op(const char* kt, int m, int cc, int col, int half) {
  const int row = 32 * m + col;
  return *reinterpret_cast<const i32x4*>(kt + row * kI8Row + swz_ki(row, 2 * cc + half) * 16);
}

// s[m][r] = int32 score * ks[key]: the reference's exact_scores without the
// query factor qs*c, which multiplies later (it is positive, so it commutes
// with the row max) (/root/reference/_int8_fwd.py:328-330).
// UKS (uniform K scale: K quantised with one scale per 128-token block, so the
// 64 keys of a tile share it): s = int32 score, and the tile's ks joins the
// query factor instead (tile_qsl), one multiply per tile instead of per score.
template <bool UKS>
__device__ __forceinline__ void scale_scores(const char* kt, const i32x16 (&si)[2], int half,
                                             f32x16 (&s)[2]) {
  const float* ksl = reinterpret_cast<const float*>(kt + kKsOffset);
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (UKS) {
#pragma unroll
        for (int j = 0; j < 4; ++j) s[m][4 * i + j] = static_cast<float>(si[m][4 * i + j]);
      } else {
        const float4 k4 = *reinterpret_cast<const float4*>(ksl + 32 * m + 8 * i + 4 * half);
        s[m][4 * i + 0] = static_cast<float>(si[m][4 * i + 0]) * k4.x;
        s[m][4 * i + 1] = static_cast<float>(si[m][4 * i + 1]) * k4.y;
        s[m][4 * i + 2] = static_cast<float>(si[m][4 * i + 2]) * k4.z;
        s[m][4 * i + 3] = static_cast<float>(si[m][4 * i + 3]) * k4.w;
      }
    }
}

// The factor of a tile's scores from scale_scores<UKS>: qs*c, times the ks
// its keys share when UKS (key 0's, in LDS behind the tile's int8 rows at
// byte ks_offset).
template <bool UKS>
__device__ __forceinline__ float tile_qsl(const char* kt, int ks_offset, float qsl) {
  if constexpr (UKS) return qsl * *reinterpret_cast<const float*>(kt + ks_offset);
  return qsl;
}

__device__ __forceinline__ void qk_i8_tile(const char* kt, const i32x4 (&qi)[4], int col, int half,
                                           i32x16 (&si)[2]) {
  const i32x16 zero = {};
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    const i32x4 a0 = ki_op(kt, 0, cc, col, half);
    const i32x4 a1 = ki_op(kt, 1, cc, col, half);
    si[0] = mfma_i8(a0, qi[cc], cc == 0 ? zero : si[0]);
    si[1] = mfma_i8(a1, qi[cc], cc == 0 ? zero : si[1]);
  }
}

// ---------------------------------------------------------- INT8 P . V path
// p_e = exp2(s*qsl - bmax) in [0, 1] for the 16 scores of key tile m, codes
// round(p_e * 127) (v_cvt_pk_u8_f32: nearest, ties to even) packed 4 per
// dword in element order; adds the 16 codes to csum (v_sad_u8 against zero:
// the byte sum, exact), so the row sum is that of the quantised P the P.V
// MFMAs multiply. (v_dot4_u32_u8 gives the same sum but, like the other dot
// instructions, does not execute beside MFMAs: 0.8% slower here.)
// negb127 = log2(127) - (tile max): the exponent yields 127 * pe directly, so
// the codes need no multiply.
__device__ __forceinline__ uint32_t probs_i8(const f32x16& s, float qsl, float negb127, i32x4& pi,
                                             uint32_t csum) {
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    uint32_t d = 0;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const float pe127 = __builtin_amdgcn_exp2f(fmaf(s[4 * w + j], qsl, negb127));
      d = __builtin_amdgcn_cvt_pk_u8_f32(pe127, j, d);
    }
    pi[w] = static_cast<int>(d);
    csum = __builtin_amdgcn_sad_u8(d, 0u, csum);
  }
  return csum;
}
constexpr float kLog2_127 = 6.98868468677216585f;  // log2(127)

// ------------------------------------------- running-max int8 P . V (RUN)
// Codes against the row's running max instead of each block's own max, so
// that the P.V products of all exact blocks accumulate in int32 with no
// per-block conversion. During the exact tiles st.m is an integer (log2
// domain) at or above every scaled score seen; st.acc holds the int32 sums
// code_p * code_v of O^T (bit for bit in the fp32 registers) and st.l the sum
// of the codes as an fp32 value, both in units of 2^st.m / 127. A unit (a
// block, or a 64-key tile) whose max exceeds st.m raises it to ceil(max) and
// scales both by 2^-(the difference): the int32 sums by an arithmetic shift
// (rounding toward -inf, less than one unit of sums of order 10^4), the code
// sum exactly (ldexp; it is split over the two lanes of a row, and small
// right after a large rise, so flooring it would bias the softmax
// denominator). Overflow: |sums| <= 127 * (code sum of the row), so while
// each lane's half of the code sum stays at most 2^23 the sums stay below
// 127 * 2^24 + 2^21 < 2^31 after one more unit (a unit of 128 keys adds less
// than 128 * 127 * 127 < 2^21); past that st.m rises by one more, for both
// lanes of the row.
constexpr float kRunLaneSumLimit = 8388608.f;  // 2^23
__device__ __forceinline__ void run_max(SoftmaxState& st, float bmax) {
  float m_new = fmaxf(st.m, ceilf(bmax));
  if (xhalf_max(st.l) > kRunLaneSumLimit) m_new += 1.f;
  const float d = m_new - st.m;  // +inf on the first unit: st.m = -inf, sums 0
  const int k = d < 31.f ? static_cast<int>(d) : 31;
  st.m = m_new;
  if (__any(k != 0)) {
    // whole-vector shifts: written per element (bit casts of vector
    // elements), clang 22 -O3 folded the 16 results into one value
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const i32x16 a = __builtin_bit_cast(i32x16, st.acc[dt]) >> k;
      st.acc[dt] = __builtin_bit_cast(f32x16, a);
    }
    st.l = __builtin_amdgcn_ldexpf(st.l, -k);
  }
}

// RUN, after the exact tiles: the int32 sums back to the fp32 state,
// O^T = sums * vscale[d] / 127 and l = code sum / 127, relative to 2^st.m.
__device__ __forceinline__ void run_finish(SoftmaxState& st, const float* vsc, int half) {
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const i32x16 a = __builtin_bit_cast(i32x16, st.acc[dt]);
#pragma unroll
    for (int r = 0; r < 16; ++r)
      st.acc[dt][r] = static_cast<float>(a[r]) *
                      (vsc[32 * dt + 8 * (r >> 2) + 4 * half + (r & 3)] * (1.f / 127.f));
  }
  st.l *= 1.f / 127.f;
}

// O^T += (Vi^T . Pi^T) * f: lane (channel 32dt + col, half) takes keys
// 32ks + 8i + 4half + j (i, j < 4) of the int8 V tile from two ds_read_tr8:
// within a 16-lane group, lane s supplies key (s >> 1) of the 8 keys read,
// channels 8(s & 1) .. +7.
// RUN: the products accumulate into the int32 sums held in acc (f unused).
template <bool RUN>
__device__ __forceinline__ void pv_i8(const char* vt, const i32x4 (&pi)[2], float f, int lane,
                                      f32x16 (&acc)[4]) {
  const i32x16 zero = {};
  const int g = lane >> 4, sl = lane & 15, half = lane >> 5;
  const int kk = sl >> 1;
  const int key_in = 8 * (kk >> 2) + 4 * half + (kk & 3);
  if constexpr (RUN) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int chunk = 2 * dt + (g & 1);
      i32x16 a32 = __builtin_bit_cast(i32x16, acc[dt]);
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int r0 = 32 * ks + key_in, r1 = r0 + 16;
        const i32x2 lo = tr8(vt + r0 * kI8Row + swz_vi(r0, chunk) * 16 + 8 * (sl & 1));
        const i32x2 hi = tr8(vt + r1 * kI8Row + swz_vi(r1, chunk) * 16 + 8 * (sl & 1));
        const i32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        a32 = mfma_i8(a, pi[ks], a32);
      }
      acc[dt] = __builtin_bit_cast(f32x16, a32);
      asm volatile("" : "+v"(acc[dt]));
    }
    return;
  }
  const auto tile = [&](int dt) {
    const int chunk = 2 * dt + (g & 1);
    i32x16 pv;
#pragma unroll
    for (int ks = 0; ks < 2; ++ks) {
      const int r0 = 32 * ks + key_in, r1 = r0 + 16;
      const i32x2 lo = tr8(vt + r0 * kI8Row + swz_vi(r0, chunk) * 16 + 8 * (sl & 1));
      const i32x2 hi = tr8(vt + r1 * kI8Row + swz_vi(r1, chunk) * 16 + 8 * (sl & 1));
      const i32x4 a = {lo[0], lo[1], hi[0], hi[1]};
      pv = mfma_i8(a, pi[ks], ks == 0 ? zero : pv);
    }
    return pv;
  };
  // The MFMAs of channel tile dt+1 run while tile dt is converted. The empty
  // asm pins each converted tile in place: left to itself the compiler issues
  // all eight MFMAs first and sinks the conversions, holding four int32
  // accumulators (64 VGPRs) at once.
  i32x16 pv[2];
  pv[0] = tile(0);
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    if (dt + 1 < 4) pv[(dt + 1) & 1] = tile(dt + 1);
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[dt][r] = fmaf(static_cast<float>(pv[dt & 1][r]), f, acc[dt][r]);
    asm volatile("" : "+v"(acc[dt]));
  }
}

// Softmax + P.V of an exact tile whose scaled scores are in s (masked keys
// already -inf): /root/reference/_int8_fwd.py:333-368. RUN: codes against
// the running max, into the int32 sums (run_max).
template <bool INT8_PV, bool RUN = false>
__device__ __forceinline__ void exact_softmax_pv(SoftmaxState& st, f32x16 (&s)[2], const void* vt,
                                                 float qsl, int lane) {
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[m][r]);
  const float bmax = xhalf_max(mx) * qsl;
  if constexpr (INT8_PV && RUN) {
    run_max(st, bmax);
    i32x4 pi[2];
    uint32_t csum = probs_i8(s[0], qsl, kLog2_127 - st.m, pi[0], 0u);
    csum = probs_i8(s[1], qsl, kLog2_127 - st.m, pi[1], csum);
    st.l += static_cast<float>(csum);
    pv_i8<true>(static_cast<const char*>(vt), pi, 0.f, lane, st.acc);
    return;
  }
  float alpha;
  st.m = new_max(st.m, bmax, alpha);
  if constexpr (INT8_PV) {
    const float beta = __builtin_amdgcn_exp2f(bmax - st.m);
    i32x4 pi[2];
    uint32_t csum = probs_i8(s[0], qsl, kLog2_127 - bmax, pi[0], 0u);
    csum = probs_i8(s[1], qsl, kLog2_127 - bmax, pi[1], csum);
    st.l = fmaf(st.l, alpha, beta * (1.f / 127.f) * static_cast<float>(csum));
    rescale(st, alpha);
    pv_i8<false>(static_cast<const char*>(vt), pi, beta * (1.f / 127.f), lane, st.acc);
  } else {
    const float neg = -st.m;
    bf16x8 pb[4];
    float psum = 0.f;
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      psum = exp8<0>(s[m], qsl, neg, pb[2 * m], psum);
      psum = exp8<8>(s[m], qsl, neg, pb[2 * m + 1], psum);
    }
    st.l = fmaf(st.l, alpha, psum);
    rescale(st, alpha);
    pv_tile(static_cast<const uint16_t*>(vt), pb, lane, st.acc);
  }
}

// Pipelined step over full exact tile n (scaled scores in sc, factor qsl):
// the i8 MFMAs of S(n+1) from the K tile kn are interleaved with the softmax
// of tile n; then P(n).V(n) and the conversion of S(n+1) into sn (ks of tile
// n+1 from kn).
// mid(): called before P(n).V(n) reads the V tile (a single-buffered V tile
// is waited for there).
// asm i8 MFMAs of the hand-ordered step (hazards as for the bf16 ones in
// fwd_common.hpp).
__device__ __forceinline__ void mfma_i8_v0(i32x16& d, const i32x4& a, const i32x4& b) {
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_i8_v(i32x16& d, const i32x4& a, const i32x4& b) {
  asm volatile("v_mfma_i32_32x32x32_i8 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}

// bf16 P.V form of the pipelined step, hand-ordered like the BF16 forward's
// steps: each of the 8 i8 score MFMAs of S(n+1) is followed by the exps of two
// P(n) words; after mid(), each of the 16 P.V MFMAs by the conversion of two
// int32 scores of S(n+1) to fp32 (times their ks). The K and V operands are
// read two MFMAs ahead, the ks one group (four scores) ahead; the lazy tile
// max is the BF16 forward's. (Spreading the exps over both phases, with the
// tile max taken every step so that the P.V MFMAs could start on the first P
// words, measured 7% slower.)
template <bool UKS, typename Mid>
__device__ __forceinline__ void fast_step_bf16pv(SoftmaxState& st, const f32x16 (&sc)[2],
                                                 f32x16 (&sn)[2], const char* kn, const void* vt,
                                                 const i32x4 (&qi)[4], float qsl, int lane,
                                                 Mid&& mid) {
  const int col = lane & 31, half = lane >> 5;
  i32x16 si[2];
  i32x4 ka[3];
  bf16x8 va[3], pb[4];
  uint32_t pw[4][4];
  float psum = 0.f;
  const float neg = -st.m;
  const uint16_t* vtile = static_cast<const uint16_t*>(vt);
  ka[0] = ki_op(kn, 0, 0, col, half);
  ka[1] = ki_op(kn, 1, 0, col, half);
  asm volatile("" ::: "memory");
  const auto unit = [&](int u) {
    const int ks = u >> 2, w = u & 3;
    const int r = 8 * (ks & 1) + 2 * w;
    pw[ks][w] = exp_pair(sc[ks >> 1][r], sc[ks >> 1][r + 1], qsl, neg, psum);
  };
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    if (i + 2 < 8) {
      ka[(i + 2) % 3] = ki_op(kn, (i + 2) & 1, (i + 2) >> 1, col, half);
      asm volatile("" ::: "memory");
    }
    if (i < 2)
      mfma_i8_v0(si[i & 1], ka[i % 3], qi[i >> 1]);
    else
      mfma_i8_v(si[i & 1], ka[i % 3], qi[i >> 1]);
    unit(2 * i);
    unit(2 * i + 1);
  }
  // the int32 scores are read after this point: 16 VALU instructions (the
  // last two exp pairs) follow the last score MFMA
  asm volatile("" : "+v"(si[0]), "+v"(si[1]));
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    pb[ks] = __builtin_bit_cast(bf16x8, make_uint4(pw[ks][0], pw[ks][1], pw[ks][2], pw[ks][3]));
  float alpha = 1.f;
  if (__any(!(psum <= 255.f))) {  // (also catches inf / NaN)
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(sc[0][r], sc[1][r]));
    const float m_new = new_max(st.m, xhalf_max(mx) * qsl, alpha);
    if (__any(m_new != st.m)) {  // lanes whose max stays recompute the same P
      st.m = m_new;
      psum = 0.f;
      psum = exp8<0>(sc[0], qsl, -m_new, pb[0], psum);
      psum = exp8<8>(sc[0], qsl, -m_new, pb[1], psum);
      psum = exp8<0>(sc[1], qsl, -m_new, pb[2], psum);
      psum = exp8<8>(sc[1], qsl, -m_new, pb[3], psum);
      mfma_fence(st.acc);  // the rescale reads O
      rescale(st, alpha);
    }
  }
  st.l = fmaf(st.l, alpha, psum);
  mid();
  // ks of score group g (elements 4(g%4) .. +3 of tile g/4): read one group
  // ahead of its two slots
  const float* ksl = reinterpret_cast<const float*>(kn + kKsOffset);
  const auto ks_group = [&](int g) {
    return *reinterpret_cast<const float4*>(ksl + 32 * (g >> 2) + 8 * (g & 3) + 4 * half);
  };
  float4 kq[2];
  if constexpr (!UKS) kq[0] = ks_group(0);
  const uint32_t vl = v_lane(lds_addr(vtile), lane);
  va[0] = v_op_x(vl, 0, 0);
  va[1] = v_op_x(vl, 0, 1);
  asm volatile("" ::: "memory");
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i + 2 < 16) {
      va[(i + 2) % 3] = v_op_x(vl, (i + 2) >> 2, (i + 2) & 3);
      if (!UKS && (i & 1) == 0 && (i >> 1) + 1 < 8) kq[((i >> 1) + 1) & 1] = ks_group((i >> 1) + 1);
      asm volatile("" ::: "memory");
    }
    if (i == 0)
      mfma_v_first(st.acc[0], va[0], pb[0]);
    else
      mfma_v(st.acc[i & 3], va[i % 3], pb[i >> 2]);
    // scores 2i, 2i + 1 of S(n+1): element e of tile m (group i/2)
#pragma unroll
    for (int t = 0; t < 2; ++t) {
      const int e2 = 2 * i + t, m = e2 >> 4, e = e2 & 15;
      const float f = static_cast<float>(si[m][e]);
      if constexpr (UKS) {
        sn[m][e] = f;
      } else {
        const float4 kk = kq[(i >> 1) & 1];
        const float kv = (e & 3) == 0 ? kk.x : (e & 3) == 1 ? kk.y : (e & 3) == 2 ? kk.z : kk.w;
        sn[m][e] = f * kv;
      }
    }
    asm volatile("" : "+v"(sn[i >> 3]));
  }
  mfma_fence(st.acc);  // O is read by plain code after the pipeline
}

// Three-stage bf16 P.V step (block 128): S(n+1) = Ki(n+1) Qi^T (8 i8 MFMAs),
// O += P(n-1) V(n-1) (16 bf16 MFMAs) and the softmax of S(n) in one
// hand-ordered stream: slot i (16) issues score MFMA i (i < 8), the exps of P
// word i, then P.V MFMA i; slots 8-15 also convert four int32 scores of S(n+1)
// to fp32 times their ks (read two slots ahead, while tile n+1's ks are in
// LDS). The last score MFMA is followed by two exp pairs and a P.V MFMA before
// the int32 scores are read. QK = false: the last tile (no scores to make);
// PV = false: the first. Lazy tile max, hazards and the final O rescale as
// in the BF16 forward's step3. qc: the factor of sc's scores.
template <bool QK, bool PV, bool UKS>
__device__ __forceinline__ void step3_i8(SoftmaxState& st, const f32x16 (&sc)[2], float qc,
                                         f32x16 (&sn)[2], const bf16x8 (&pp)[4], bf16x8 (&pn)[4],
                                         const char* kn, uint32_t vl, const i32x4 (&qi)[4],
                                         int lane) {
  const int col = lane & 31, half = lane >> 5;
  i32x16 si[2];
  i32x4 ka[3];
  bf16x8 va[3];
  float4 kq[3];
  uint32_t pw[4][4];
  float psum = 0.f;
  const float neg = -st.m;
  const float* ksl = QK ? reinterpret_cast<const float*>(kn + kKsOffset) : nullptr;
  const auto ks_group = [&](int g) {
    return *reinterpret_cast<const float4*>(ksl + 32 * (g >> 2) + 8 * (g & 3) + 4 * half);
  };
  if constexpr (QK) {
    ka[0] = ki_op(kn, 0, 0, col, half);
    ka[1] = ki_op(kn, 1, 0, col, half);
  }
  if constexpr (PV) {
    va[0] = v_op_x(vl, 0, 0);
    va[1] = v_op_x(vl, 0, 1);
  }
  asm volatile("" ::: "memory");
  const auto unit = [&](int u) {
    const int ks = u >> 2, w = u & 3;
    const int r = 8 * (ks & 1) + 2 * w;
    pw[ks][w] = exp_pair(sc[ks >> 1][r], sc[ks >> 1][r + 1], qc, neg, psum);
  };
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if constexpr (QK) {
      if (i + 2 < 8) ka[(i + 2) % 3] = ki_op(kn, (i + 2) & 1, (i + 2) >> 1, col, half);
      if (!UKS && i >= 6 && i <= 13) kq[(i - 6) % 3] = ks_group(i - 6);
    }
    if constexpr (PV) {
      if (i + 2 < 16) va[(i + 2) % 3] = v_op_x(vl, (i + 2) >> 2, (i + 2) & 3);
    }
    asm volatile("" ::: "memory");
    if constexpr (QK) {
      if (i < 2)
        mfma_i8_v0(si[i & 1], ka[i % 3], qi[i >> 1]);
      else if (i < 8)
        mfma_i8_v(si[i & 1], ka[i % 3], qi[i >> 1]);
    }
    unit(i);
    if constexpr (PV) {
      if (i == 0)
        mfma_v_first(st.acc[0], va[0], pp[0]);
      else
        mfma_v(st.acc[i & 3], va[i % 3], pp[i >> 2]);
    }
    if constexpr (QK) {
      if (i == 8) asm volatile("" : "+v"(si[0]), "+v"(si[1]));  // the int32 scores are read after this
      if (i >= 8) {
        const int g = i - 8, m = g >> 2, e0 = 4 * (g & 3);
        const float4 kk = kq[g % 3];
#pragma unroll
        for (int t = 0; t < 4; ++t) {
          const float f = static_cast<float>(si[m][e0 + t]);
          if constexpr (UKS) {
            sn[m][e0 + t] = f;
          } else {
            const float kv = t == 0 ? kk.x : t == 1 ? kk.y : t == 2 ? kk.z : kk.w;
            sn[m][e0 + t] = f * kv;
          }
        }
        asm volatile("" : "+v"(sn[m]));
      }
    }
    if (i == 0) __builtin_amdgcn_s_setprio(1);
  }
  __builtin_amdgcn_s_setprio(0);
  if constexpr (!QK) mfma_fence(st.acc);  // the plain path's builtin MFMAs follow
#pragma unroll
  for (int ks = 0; ks < 4; ++ks)
    pn[ks] = __builtin_bit_cast(bf16x8, make_uint4(pw[ks][0], pw[ks][1], pw[ks][2], pw[ks][3]));
  float alpha = 1.f;
  if (__any(!(psum <= 255.f))) {  // (also catches inf / NaN)
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(sc[0][r], sc[1][r]));
    const float m_new = new_max(st.m, xhalf_max(mx) * qc, alpha);
    if (__any(m_new != st.m)) {  // lanes whose max stays recompute the same P
      st.m = m_new;
      psum = 0.f;
      psum = exp8<0>(sc[0], qc, -m_new, pn[0], psum);
      psum = exp8<8>(sc[0], qc, -m_new, pn[1], psum);
      psum = exp8<0>(sc[1], qc, -m_new, pn[2], psum);
      psum = exp8<8>(sc[1], qc, -m_new, pn[3], psum);
      if constexpr (PV) mfma_fence(st.acc);  // the rescale reads O
      rescale(st, alpha);
    }
  }
  st.l = fmaf(st.l, alpha, psum);
}

template <bool INT8_PV, bool UKS, bool RUN, typename Mid>
__device__ __forceinline__ void fast_step(SoftmaxState& st, f32x16 (&sc)[2], f32x16 (&sn)[2],
                                          const char* kn, const void* vt, const i32x4 (&qi)[4],
                                          float qsl, int lane, Mid&& mid) {
  if constexpr (!INT8_PV) {
    fast_step_bf16pv<UKS>(st, sc, sn, kn, vt, qi, qsl, lane, mid);
    return;
  }
  const int col = lane & 31, half = lane >> 5;
  const i32x16 zero = {};
  i32x16 si[2];
  i32x4 ka[4][2];
  // bf16 P.V: lazy tile max, as in the BF16 forward's steps (the exps use the
  // running max as it stands; the tile max is taken only when a lane's row
  // sum exceeds 255, or is inf on a first tile with the running max -inf), so
  // the running max evolves as if taken every tile. int8 P.V needs the block
  // max itself: its P codes are relative to it (RUN: to the running max).
  float mx = -INFINITY, alpha = 1.f, bmax = 0.f, neg = INT8_PV ? 0.f : -st.m, psum = 0.f;
  uint32_t csum = 0u;
  bf16x8 pb[4];
  i32x4 pi[2];
  ka[0][0] = ki_op(kn, 0, 0, col, half);
  ka[0][1] = ki_op(kn, 1, 0, col, half);
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) {
    if (cc + 1 < 4) {
      ka[cc + 1][0] = ki_op(kn, 0, cc + 1, col, half);
      ka[cc + 1][1] = ki_op(kn, 1, cc + 1, col, half);
    }
    si[0] = mfma_i8(ka[cc][0], qi[cc], cc == 0 ? zero : si[0]);
    si[1] = mfma_i8(ka[cc][1], qi[cc], cc == 0 ? zero : si[1]);
    if (cc == 0 && INT8_PV) {
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[m][r]);
      bmax = xhalf_max(mx) * qsl;
      if constexpr (RUN) {
        run_max(st, bmax);
        bmax = st.m;  // the codes' reference
      } else {
        st.m = new_max(st.m, bmax, alpha);
      }
      neg = -st.m;
    } else if (cc == 1) {
      if constexpr (INT8_PV) {
        csum = probs_i8(sc[0], qsl, kLog2_127 - bmax, pi[0], csum);
      } else {
        psum = exp8<0>(sc[0], qsl, neg, pb[0], psum);
        psum = exp8<8>(sc[0], qsl, neg, pb[1], psum);
      }
    } else if (cc == 2) {
      if constexpr (INT8_PV) {
        csum = probs_i8(sc[1], qsl, kLog2_127 - bmax, pi[1], csum);
      } else {
        psum = exp8<0>(sc[1], qsl, neg, pb[2], psum);
        psum = exp8<8>(sc[1], qsl, neg, pb[3], psum);
        if (__any(!(psum <= 255.f))) {
#pragma unroll
          for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(sc[0][r], sc[1][r]));
          const float m_new = new_max(st.m, xhalf_max(mx) * qsl, alpha);
          if (__any(m_new != st.m)) {  // lanes whose max stays recompute the same P
            st.m = m_new;
            neg = -m_new;
            psum = 0.f;
            psum = exp8<0>(sc[0], qsl, neg, pb[0], psum);
            psum = exp8<8>(sc[0], qsl, neg, pb[1], psum);
            psum = exp8<0>(sc[1], qsl, neg, pb[2], psum);
            psum = exp8<8>(sc[1], qsl, neg, pb[3], psum);
          }
        }
      }
    }
  }
  float beta = 1.f;
  if constexpr (INT8_PV && RUN) {
    st.l += static_cast<float>(csum);
  } else if constexpr (INT8_PV) {
    beta = __builtin_amdgcn_exp2f(bmax - st.m);
    st.l = fmaf(st.l, alpha, beta * (1.f / 127.f) * static_cast<float>(csum));
  } else {
    st.l = fmaf(st.l, alpha, psum);
  }
  if constexpr (!RUN) rescale(st, alpha);
  if constexpr (INT8_PV) {
    scale_scores<UKS>(kn, si, half, sn);  // frees the int32 scores before the P.V accumulators
    mid();
    pv_i8<RUN>(static_cast<const char*>(vt), pi, beta * (1.f / 127.f), lane, st.acc);
  } else {
    mid();
    pv_tile(static_cast<const uint16_t*>(vt), pb, lane, st.acc);
    scale_scores<UKS>(kn, si, half, sn);
  }
}

// ------------------------------------------------------------------ copies
struct I8Source {
  const int8_t* ki;  // rows of this batch/head, stride srow bytes
  const float* ks;   // this head's scales, kst floats from token to token
  const int8_t* vi;
  int64_t srow;
  int kst;
};

// Per-lane byte offsets of this lane's 16-byte chunk of an int8 tile (copy u
// adds (NTHREADS/8) u rows; the swizzles repeat, so one offset per tile kind).
template <int NTHREADS>
struct I8Offsets {
  static constexpr int U = kKeys * 8 / NTHREADS;  // copies per lane per int8 tile
  static constexpr int kKsPerWave = kKeys / (NTHREADS / 64);
  uint32_t k, v, ks;  // ks: this lane's key of the tile (waves copy kKsPerWave each) x kst x 4
  __device__ __forceinline__ void init(int64_t srow, int kst) {
    const int row = threadIdx.x >> 3, pc = threadIdx.x & 7;
    k = static_cast<uint32_t>(row * srow + swz_ki(row, pc) * 16);
    v = static_cast<uint32_t>(row * srow + swz_vi(row, pc) * 16);
    const int key = kKsPerWave * (threadIdx.x >> 6) + (threadIdx.x & 63);
    ks = static_cast<uint32_t>(key * kst * 4);
  }
};

// int8 rows [first, first + 64) (rows past nvalid re-read row 0 when !FULL)
// of ki (or vi) into an LDS tile; with KS also the 64 ks, each wave copying
// 64 / nwaves of them.
template <int NTHREADS, bool FULL, bool KS>
__device__ __forceinline__ void issue_i8(uint32_t dst, const int8_t* rows, const I8Source& is, int first,
                                         int nvalid, uint32_t off, uint32_t ks_off, bool is_v) {
  constexpr int U = I8Offsets<NTHREADS>::U;
  const uint32_t l0 = dst;
  const int wave = wave_id();
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const uint32_t d = l0 + (wave * 64 + NTHREADS * u) * 16;
    if constexpr (FULL) {
      const char* base = reinterpret_cast<const char*>(rows) +
                         static_cast<int64_t>(first + u * (NTHREADS / 8)) * is.srow;
      g2l16_s(base, off, d);
    } else {
      const int e = threadIdx.x + NTHREADS * u;
      const int row = e >> 3, pc = e & 7;
      const int srow = first + (row < nvalid ? row : 0);
      const int chunk = is_v ? swz_vi(row, pc) : swz_ki(row, pc);
      g2l16(reinterpret_cast<const char*>(rows) + static_cast<int64_t>(srow) * is.srow + chunk * 16, d);
    }
  }
  if constexpr (KS) {
    constexpr int kpw = I8Offsets<NTHREADS>::kKsPerWave;
    const int lane = threadIdx.x & 63;
    if (lane < kpw) {
      const uint32_t d = l0 + kKsOffset + 4 * kpw * wave;
      if constexpr (FULL) {
        g2l4_s(is.ks + static_cast<int64_t>(first) * is.kst, ks_off, d);
      } else {
        const int key = kpw * wave + lane;
        const int r = key < nvalid ? key : 0;
        g2l4(is.ks + static_cast<int64_t>(first + r) * is.kst, d);
      }
    }
  }
}

// K and V tiles double buffered. Block 128: 68 KB of LDS, two workgroups per
// CU, two waves per SIMD. Block 64: packed int8 K tiles, double buffered; with
// int8 P.V packed int8 V too, double buffered (37 KB, four workgroups per CU),
// with bf16 P.V one bf16 V tile (VSINGLE: 36 KB, four workgroups per CU, two
// waves on every SIMD), copied after the step's P.V and waited for before the
// next one's.
template <int BLK, bool INT8_PV, bool UKS, bool RUN>
__global__ void __launch_bounds__(BLK * 2)
__attribute__((amdgpu_waves_per_eu(2)))
fwd_int8_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                const int8_t* __restrict__ qi, const float* __restrict__ qs,
                const int8_t* __restrict__ ki, const float* __restrict__ ks,
                const int8_t* __restrict__ vi, const float* __restrict__ vscale,
                const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                int64_t TP, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                int64_t npad, const int32_t* __restrict__ counts, const uint32_t* __restrict__ mask, int T, int H, int NT, int W, float c,
                uint16_t* __restrict__ o, int64_t so_b, int64_t so_t, int64_t so_h, int kst,
                int64_t ksh) {
  constexpr int NTHREADS = BLK * 2;
  // LDS: exact-tile buffers K(i), V(i), i < 2. COMPACT (block 64): the int8
  // tiles are packed (K + its ks: 8448 B; int8 V: 8192 B), so with int8 P.V two
  // of each take 33 KB and four workgroups fit a CU, with bf16 P.V (16 KB V
  // tiles) 49 KB and three; a bf16 pooled tile then spans K(0)-K(1) (and, with
  // int8 P.V, V(0)-V(1)) and the pooled tiles are single buffered.
  constexpr int NBUF = 2;
  constexpr bool COMPACT = BLK == 64;
  constexpr bool VSINGLE = COMPACT && !INT8_PV;  // one bf16 V tile buffer
  constexpr int NVBUF = VSINGLE ? 1 : NBUF;
  constexpr int KSTRIDE = COMPACT ? kKsOffset + 256 : static_cast<int>(kTileBytes);
  constexpr int VSTRIDE = COMPACT && INT8_PV ? kKeys * kD : static_cast<int>(kTileBytes);
  constexpr int VBASE = NBUF * KSTRIDE;
  constexpr int PNBUF = COMPACT ? 1 : NBUF;  // buffers for pooled tiles
  static_assert(!COMPACT || (2 * KSTRIDE >= static_cast<int>(kTileBytes) &&
                             NVBUF * VSTRIDE >= static_cast<int>(kTileBytes)), "pooled tile must fit");
  // copies per wave of one K tile (rows and ks): VSINGLE waits for the V tile
  // issued before them with these still in flight
  constexpr int kKCopies = I8Offsets<NTHREADS>::U + 1;
  __shared__ __align__(256) char arena[VBASE + NVBUF * VSTRIDE];
  __shared__ TileList tl;
  const auto Kp = [&](int i) { return reinterpret_cast<uint16_t*>(arena + i * KSTRIDE); };
  const auto Vp = [&](int i) {
    return reinterpret_cast<uint16_t*>(arena + VBASE + (VSINGLE ? 0 : i) * VSTRIDE);
  };
  const auto bi = [](int n) { return n & 1; };                      // buffer of exact tile n
  const auto bp = [](int n) { return PNBUF == 2 ? (n & 1) : 0; };   // buffer of pooled tile n

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  int bh, qb;
  tile_coords_lpt<kLptTokens / BLK>(counts, NT, bh, qb);
  const int b = bh / H, h = bh % H;
  const int64_t row = static_cast<int64_t>(bh) * NT + qb;

  const int ntiles = build_tile_list<BLK>(tl, mask, row, NT, W, T);
  if (ntiles == 0) return;  // cannot happen for routed masks: the diagonal is exact
  const int nrag = ragged_tiles(tl, NT, T);
  const int nexact = tl.nexact;       // tiles [0, nexact): ragged first, then full
  const int nfast = nexact - nrag;    // tiles [nexact, ntiles): pooled

  const int64_t bhD = (static_cast<int64_t>(b) * npad * H + h) * kD;
  const KVSource src{nullptr, 0, v + b * sv_b + h * sv_h, sv_t, kc + bhD,
                     static_cast<int64_t>(H) * kD, vc + bhD};
  const I8Source is{ki + (static_cast<int64_t>(b) * TP * H + h) * kD,
                    ks + static_cast<int64_t>(b) * TP * H + h * ksh,
                    vi + (static_cast<int64_t>(b) * TP * H + h) * kD,
                    static_cast<int64_t>(H) * kD, kst};
  I8Offsets<NTHREADS> ioff;
  ioff.init(is.srow, kst);
  CopyOffsets<NTHREADS> boff;
  boff.init(0, sv_t);

  // Exact tile n of this kernel's order: n < nrag is the ragged one (list
  // tile nexact - 1), then list tiles 0 .. nfast-1.
  const auto exact_tile = [&](int n) {
    return exact_desc<BLK>(tl, n < nrag ? nexact - 1 : n - nrag, T, NT);
  };
  const uint32_t kb = lds_addr(arena), vb = kb + VBASE;  // LDS byte addresses
  const auto kbuf_at = [&](int buf) { return kb + buf * KSTRIDE; };
  const auto vbuf_at = [&](int buf) { return vb + (VSINGLE ? 0 : buf) * VSTRIDE; };
  const auto issue_exact_full = [&](int n, uint32_t kd, uint32_t vd, bool with_k, bool with_v) {
    const int first = exact_first<BLK>(tl, n - nrag);
    if (with_k) issue_i8<NTHREADS, true, true>(kd, is.ki, is, first, kKeys, ioff.k, ioff.ks, false);
    if (with_v) {
      if constexpr (INT8_PV)
        issue_i8<NTHREADS, true, false>(vd, is.vi, is, first, kKeys, ioff.v, 0, true);
      else
        issue_full<NTHREADS>(vd, src.v + static_cast<int64_t>(first) * src.sv, src.sv, boff.v);
    }
  };
  const auto issue_tile = [&](int n, int buf) {
    const uint32_t kd = kbuf_at(buf), vd = vbuf_at(buf);
    if (n >= nexact) {
      const TileDesc td = pooled_desc(tl, n - nexact, NT);
      issue_generic<NTHREADS>(kd, 0, td, src);
      issue_generic<NTHREADS>(vd, 1, td, src);
    } else if (n >= nrag) {
      issue_exact_full(n, kd, vd, true, true);
    } else {
      const TileDesc td = exact_tile(n);
      issue_i8<NTHREADS, false, true>(kd, is.ki, is, td.first, td.nvalid, 0, 0, false);
      if constexpr (INT8_PV)
        issue_i8<NTHREADS, false, false>(vd, is.vi, is, td.first, td.nvalid, 0, 0, true);
      else
        issue_generic<NTHREADS>(vd, 1, td, src);
    }
  };
  issue_tile(0, 0);

  const int qrow = qb * BLK + wave * 32 + col;
  const bool qvalid = qrow < T;
  SoftmaxState st;
  st.init();

  // ---- exact tiles (int8 Q: 16 VGPRs)
  if (nexact > 0) {
    i32x4 qireg[4];
    float qsl = 0.f;
    {
      const int64_t qoff = (static_cast<int64_t>(b) * TP + qrow) * H + h;
      const int8_t* qip = qi + qoff * kD + half * 16;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        uint4 r = make_uint4(0u, 0u, 0u, 0u);
        if (qvalid) r = *reinterpret_cast<const uint4*>(qip + cc * 32);
        qireg[cc] = __builtin_bit_cast(i32x4, r);
      }
      if (qvalid) qsl = qs[qoff] * c;
    }
    // ragged tile: plain, masked
    if (nrag) {
      wait_tile_copies();
      __syncthreads();
      // a pooled tile 1 does not fit buffer 1 when COMPACT: the pooled phase
      // issues it; VSINGLE: tile 1's V follows the ragged tile's P.V
      if (1 < ntiles && (!COMPACT || 1 < nexact)) {
        if constexpr (VSINGLE)
          issue_exact_full(1, kbuf_at(1), 0u, true, false);
        else
          issue_tile(1, 1);
      }
      const TileDesc td = exact_tile(0);
      i32x16 si[2];
      f32x16 s[2];
      const char* kt = reinterpret_cast<const char*>(Kp(0));
      qk_i8_tile(kt, qireg, col, half, si);
      scale_scores<UKS>(kt, si, half, s);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t bits = static_cast<uint32_t>(td.amask >> (32 * m + 4 * half));
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s[m][r] = ((bits >> (8 * (r >> 2) + (r & 3))) & 1u) ? s[m][r] : -INFINITY;
      }
      exact_softmax_pv<INT8_PV, RUN>(st, s, Vp(0), tile_qsl<UKS>(kt, kKsOffset, qsl), lane);
      __syncthreads();
      if constexpr (VSINGLE) {
        if (1 < nexact) issue_exact_full(1, 0u, vbuf_at(0), false, true);
      }
    }
    // full exact tiles, pipelined (tile F = nrag was issued into buffers bi(F));
    // fa, fb: the score factors of sa, sb
    const int F = nrag;
    if (nfast > 0) {
      const int E = nexact;  // one past the last full exact tile
      f32x16 sa[2], sb[2];
      float fa, fb;
      const auto qk_scaled = [&](const uint16_t* kb, f32x16 (&s)[2]) {
        i32x16 si[2];
        const char* kt = reinterpret_cast<const char*>(kb);
        qk_i8_tile(kt, qireg, col, half, si);
        scale_scores<UKS>(kt, si, half, s);
        return tile_qsl<UKS>(kt, kKsOffset, qsl);
      };
      wait_tile_copies();
      __syncthreads();
      if (F + 1 < E) issue_exact_full(F + 1, kbuf_at((F + 1) & 1), 0u, true, false);
      fa = qk_scaled(Kp(F & 1), sa);
      wait_tile_copies();
      __syncthreads();  // K(F & 1) is refilled (K of tile F+2) by the first step
      int n = F;
      if constexpr (!INT8_PV && !VSINGLE) {
        // Three-stage pipeline (step3_i8). On entry to step n (F < n < E-1):
        // S(n) and P(n-1) in registers, K(n+1) and V(n-1) in LDS; the step
        // copies K(n+2) over K(n) and V(n) over V(n-2) (V(F) came with tile F).
        const uint32_t vl0 = v_lane(vbuf_at(0), lane);
        if (F + 1 < E) {
          bf16x8 pa[4], pb[4];
          issue_exact_full(min(F + 2, E - 1), kbuf_at(F & 1), 0u, true, false);
          {
            const char* kn = reinterpret_cast<const char*>(Kp((F + 1) & 1));
            step3_i8<true, false, UKS>(st, sa, fa, sb, pb, pa, kn, 0u, qireg, lane);
            fb = tile_qsl<UKS>(kn, kKsOffset, qsl);
          }
          wait_tile_copies();
          __syncthreads();
          n = F + 1;  // S(n) in sb (factor fb), P(n-1) in pa
          const auto gstep = [&](const f32x16 (&sc)[2], float fc, f32x16 (&sn)[2], float& fnext,
                                 const bf16x8 (&pp)[4], bf16x8 (&pn)[4]) {
            issue_exact_full(min(n + 2, E - 1), kbuf_at(n & 1), 0u, true, false);
            issue_exact_full(n, 0u, vbuf_at(n & 1), false, true);
            const char* kn = reinterpret_cast<const char*>(Kp((n + 1) & 1));
            step3_i8<true, true, UKS>(st, sc, fc, sn, pp, pn, kn, vl0 + ((n - 1) & 1) * VSTRIDE,
                                      qireg, lane);
            fnext = tile_qsl<UKS>(kn, kKsOffset, qsl);
            wait_tile_copies();
            __syncthreads();
            ++n;
          };
          const auto last = [&](const f32x16 (&sc)[2], float fc, f32x16 (&dummy)[2],
                                const bf16x8 (&pp)[4], bf16x8 (&pn)[4]) {
            issue_exact_full(n, 0u, vbuf_at(n & 1), false, true);  // V(E-1)
            step3_i8<false, true, UKS>(st, sc, fc, dummy, pp, pn, nullptr,
                                       vl0 + ((n - 1) & 1) * VSTRIDE, qireg, lane);
            wait_tile_copies();
            __syncthreads();
            pv_tile(reinterpret_cast<const uint16_t*>(Vp(n & 1)), pn, lane, st.acc);
          };
          while (n + 2 < E) {
            gstep(sb, fb, sa, fa, pa, pb);
            gstep(sa, fa, sb, fb, pb, pa);
          }
          if (n + 1 < E) {
            gstep(sb, fb, sa, fa, pa, pb);
            last(sa, fa, sb, pb, pa);
          } else {
            last(sb, fb, sa, pa, pb);
          }
        } else {
          exact_softmax_pv<INT8_PV, RUN>(st, sa, Vp(bi(n)), fa, lane);
        }
        __syncthreads();
      } else {
      // Step n needs n + 1 < E. K(n+2) of the last step is clamped to the
      // last full tile: a redundant copy into a buffer nothing reads afterwards.
      // VSINGLE: V(n) was copied at the end of step n-1, before this step's
      // K(n+2); it is waited for before P(n).V(n), and V(n+1) is copied once
      // every wave is past P(n).V(n).
      const auto step = [&](f32x16 (&sc)[2], float qc, f32x16 (&sn)[2], float& qn) {
        issue_exact_full(min(n + 2, E - 1), kbuf_at(n & 1), 0u, true, false);
        if constexpr (!VSINGLE) issue_exact_full(n + 1, 0u, vbuf_at((n + 1) & 1), false, true);
        const char* kn = reinterpret_cast<const char*>(Kp((n + 1) & 1));
        fast_step<INT8_PV, UKS, RUN>(st, sc, sn, kn, Vp(n & 1), qireg, qc, lane, [&] {
          if constexpr (VSINGLE) {
            wait_vmcnt<kKCopies>();
            __syncthreads();
          }
        });
        qn = tile_qsl<UKS>(kn, kKsOffset, qsl);
        wait_tile_copies();
        __syncthreads();
        if constexpr (VSINGLE) issue_exact_full(n + 1, 0u, vbuf_at(0), false, true);
        ++n;
      };
      while (n + 2 < E) {
        step(sa, fa, sb, fb);
        step(sb, fb, sa, fa);
      }
      if constexpr (VSINGLE) {
        const bool odd = n + 1 < E;  // one more step, the last tile's scores in sb
        if (odd) step(sa, fa, sb, fb);
        wait_tile_copies();  // V of the last tile
        __syncthreads();
        if (odd)
          exact_softmax_pv<INT8_PV, RUN>(st, sb, Vp(bi(n)), fb, lane);
        else
          exact_softmax_pv<INT8_PV, RUN>(st, sa, Vp(bi(n)), fa, lane);
      } else if (n + 1 < E) {
        step(sa, fa, sb, fb);
        exact_softmax_pv<INT8_PV, RUN>(st, sb, Vp(bi(n)), fb, lane);
      } else {
        exact_softmax_pv<INT8_PV, RUN>(st, sa, Vp(bi(n)), fa, lane);
      }
      __syncthreads();
      }
    }
    if constexpr (INT8_PV) {
      // The per-channel V scale, common to every exact tile. The empty asm
      // keeps its 64 loads here: hoisted above the exact tiles they would
      // hold 64 VGPRs through the whole pipeline.
      const float* vsc = vscale + static_cast<int64_t>(bh) * kD;
      asm volatile("" : "+s"(vsc));
      if constexpr (RUN) {
        run_finish(st, vsc, half);
      } else {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) st.acc[dt][r] *= vsc[32 * dt + 8 * (r >> 2) + 4 * half + (r & 3)];
      }
    }
  }

  // ---- pooled tiles (bf16 Q: 32 VGPRs)
  if (nexact < ntiles) {
    bf16x8 qreg[8];
    const uint16_t* qp = q + b * sq_b + static_cast<int64_t>(qrow) * sq_t + h * sq_h + half * 8;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      uint4 r = make_uint4(0u, 0u, 0u, 0u);
      if (qvalid) r = *reinterpret_cast<const uint4*>(qp + cc * 16);
      qreg[cc] = __builtin_bit_cast(bf16x8, r);
    }
    if (nexact > 0) issue_tile(nexact, bp(nexact));  // every earlier copy has landed
    for (int n = nexact; n < ntiles; ++n) {
      wait_tile_copies();  // tile n: the only copies in flight
      __syncthreads();
      if constexpr (PNBUF == 2) {
        if (n + 1 < ntiles) issue_tile(n + 1, (n + 1) & 1);
      }
      f32x16 s[2];
      qk_tile(Kp(bp(n)), qreg, col, half, s);
      finish_tile<BLK>(st, s, Vp(bp(n)), pooled_desc(tl, n - nexact, NT), c, lane, NT, T);
      __syncthreads();
      if constexpr (PNBUF == 1) {
        if (n + 1 < ntiles) issue_tile(n + 1, 0);
      }
    }
  }
  wait_tile_copies();
  store_rows(st, o + b * so_b + h * so_h, so_t, qrow, T, half);
}

// ------------------------------------------- block 128 with int8 P.V
// The unit of work is the routed block of 128 keys, as in the reference at
// block 128 (/root/reference/_int8_fwd.py:333-353): P is quantised against the
// row max over the whole block, and its 128 products per channel accumulate in
// int32 before one conversion (half the conversions of two 64-key tiles).
// K block in LDS: 128 int8 rows (XOR-swizzled as the tiles) with the 128 ks
// behind them; V block: 128 int8 rows.
constexpr int kBlkKsOffset = 2 * kKsOffset;            // 16384
constexpr int kBlkKStride = kBlkKsOffset + 2 * 256;    // + 128 ks = 16896
constexpr int kBlkVStride = 2 * kKsOffset;             // 16384

// int8 rows [first, first + 128) of ki (KS: with their ks) or vi into an LDS
// block; 256 threads, four 16-byte copies per lane, each wave copying 32 ks.
template <bool KS>
__device__ __forceinline__ void issue_blk(uint32_t dst, const int8_t* rows, const I8Source& is,
                                          int first, uint32_t off, uint32_t ks_off) {
  const int wave = wave_id();
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    const char* base = reinterpret_cast<const char*>(rows) + static_cast<int64_t>(first + 32 * u) * is.srow;
    g2l16_s(base, off, dst + (wave * 64 + 256 * u) * 16);
  }
  if constexpr (KS) {
    if ((threadIdx.x & 63) < 32)
      g2l4_s(is.ks + static_cast<int64_t>(first) * is.kst, ks_off, dst + kBlkKsOffset + 128 * wave);
  }
}

// s = int32 scores of 32-key chunk m * ks[key] (UKS: the 128 keys of the
// block share one ks, which tile_qsl folds into the block's factor).
template <bool UKS>
__device__ __forceinline__ void scale_chunk(const char* kt, const i32x16& si, int m, int half, f32x16& s) {
  const float* ksl = reinterpret_cast<const float*>(kt + kBlkKsOffset) + 32 * m + 4 * half;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    if constexpr (UKS) {
#pragma unroll
      for (int j = 0; j < 4; ++j) s[4 * i + j] = static_cast<float>(si[4 * i + j]);
    } else {
      const float4 k4 = *reinterpret_cast<const float4*>(ksl + 8 * i);
      s[4 * i + 0] = static_cast<float>(si[4 * i + 0]) * k4.x;
      s[4 * i + 1] = static_cast<float>(si[4 * i + 1]) * k4.y;
      s[4 * i + 2] = static_cast<float>(si[4 * i + 2]) * k4.z;
      s[4 * i + 3] = static_cast<float>(si[4 * i + 3]) * k4.w;
    }
  }
}

// scale_chunk over the four 32-key chunks of a block.
template <bool UKS>
__device__ __forceinline__ void scale_block(const char* kt, const i32x16 (&si)[4], int half,
                                            f32x16 (&s)[4]) {
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    if (m > 0) asm volatile("" ::: "memory");  // one chunk's ks loads at a time
    scale_chunk<UKS>(kt, si[m], m, half, s[m]);
  }
}

// int32 scores of 32-key chunk m of a K block.
__device__ __forceinline__ i32x16 qk_chunk(const char* kt, const i32x4 (&qi)[4], int m, int col,
                                           int half) {
  const i32x16 zero = {};
  i32x16 si;
#pragma unroll
  for (int cc = 0; cc < 4; ++cc) si = mfma_i8(ki_op(kt, m, cc, col, half), qi[cc], cc == 0 ? zero : si);
  return si;
}

// O^T += (Vi^T . Pi^T) * f over the 128 keys of a block (4 MFMAs per channel
// tile into one int32 accumulator); lane layout as pv_i8. RUN: the MFMAs
// accumulate into the int32 sums held in acc (f unused).
template <bool RUN, typename Mid>
__device__ __forceinline__ void pv_blk(const char* vt, const i32x4 (&pi)[4], float f, int lane,
                                       f32x16 (&acc)[4], Mid&& mid) {
  const i32x16 zero = {};
  const int g = lane >> 4, sl = lane & 15, half = lane >> 5;
  const int kk = sl >> 1;
  const int key_in = 8 * (kk >> 2) + 4 * half + (kk & 3);
  const auto tile = [&](int dt, i32x16 pv, bool first) {
    const int chunk = 2 * dt + (g & 1);
#pragma unroll
    for (int ks = 0; ks < 4; ++ks) {
      const int r0 = 32 * ks + key_in, r1 = r0 + 16;
      const i32x2 lo = tr8(vt + r0 * kI8Row + swz_vi(r0, chunk) * 16 + 8 * (sl & 1));
      const i32x2 hi = tr8(vt + r1 * kI8Row + swz_vi(r1, chunk) * 16 + 8 * (sl & 1));
      const i32x4 a = {lo[0], lo[1], hi[0], hi[1]};
      pv = mfma_i8(a, pi[ks], ks == 0 && first ? zero : pv);
    }
    return pv;
  };
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    if constexpr (RUN) {
      const i32x16 pv = tile(dt, __builtin_bit_cast(i32x16, acc[dt]), false);
      mid(dt);
      acc[dt] = __builtin_bit_cast(f32x16, pv);
    } else {
      const i32x16 pv = tile(dt, zero, true);
      mid(dt);  // independent VALU work beside this tile's MFMAs
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] = fmaf(static_cast<float>(pv[r]), f, acc[dt][r]);
    }
    asm volatile("" : "+v"(acc[dt]));
  }
}

// Block step: the i8 MFMAs of S(b+1) (chunk 0 beside the row max of block b,
// chunks 1-2 beside its P codes), then P(b).V(b) and the conversion of
// S(b+1) into scaled scores while block b+1's ks are in LDS. QK = false: the
// last block (softmax and P.V only). qsl: the factor of sc's scores. RUN:
// codes against the running max, into the int32 sums (run_max).
template <bool QK, bool UKS, bool RUN>
__device__ __forceinline__ void block_step(SoftmaxState& st, const f32x16 (&sc)[4], f32x16 (&sn)[4],
                                           const char* kn, const char* vt, const i32x4 (&qi)[4],
                                           float qsl, int lane) {
  const int col = lane & 31, half = lane >> 5;
  i32x16 si[4];
  i32x4 pi[4];
  float mx = -INFINITY, alpha = 1.f, bmax = 0.f;
  uint32_t csum = 0u;
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    // the K operand reads of chunk m stay behind the work of slot m - 1, so
    // at most two chunks of S(b+1) are live beside S(b)
    if (m > 0) asm volatile("" ::: "memory");
    if constexpr (QK) si[m] = qk_chunk(kn, qi, m, col, half);
    if (m == 0) {
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) mx = fmaxf(mx, sc[j][r]);
      bmax = xhalf_max(mx) * qsl;
      if constexpr (RUN) {
        run_max(st, bmax);
        bmax = st.m;  // the codes' reference
      } else {
        st.m = new_max(st.m, bmax, alpha);
      }
    } else if (m < 3) {
      // codes of chunks 2(m-1), 2(m-1)+1; the empty asm keeps them in this
      // slot, so S(b) dies while S(b+1) accumulates
      const int j0 = 2 * (m - 1);
      csum = probs_i8(sc[j0], qsl, kLog2_127 - bmax, pi[j0], csum);
      csum = probs_i8(sc[j0 + 1], qsl, kLog2_127 - bmax, pi[j0 + 1], csum);
      asm volatile("" : "+v"(pi[j0]), "+v"(pi[j0 + 1]), "+v"(csum));
    }
  }
  float beta = 1.f;
  if constexpr (RUN) {
    st.l += static_cast<float>(csum);
  } else {
    beta = __builtin_amdgcn_exp2f(bmax - st.m);
    st.l = fmaf(st.l, alpha, beta * (1.f / 127.f) * static_cast<float>(csum));
    rescale(st, alpha);
  }
  // P(b).V(b); chunk dt of S(b+1) is scaled beside channel tile dt's MFMAs
  pv_blk<RUN>(vt, pi, beta * (1.f / 127.f), lane, st.acc, [&](int dt) {
    if constexpr (QK) {
      scale_chunk<UKS>(kn, si[dt], dt, half, sn[dt]);
      asm volatile("" : "+v"(sn[dt]));
    }
  });
}

// Block 128, int8 P.V: full exact blocks pipelined (step b: copies of K(b+2)
// and V(b+1); S(b+1) beside the softmax of block b; P(b).V(b)), then the
// tiles of a ragged last block (plain, per 64-key tile), the V channel scale,
// then the pooled tiles in bf16. K and V blocks double buffered: 65 KB of
// LDS, two workgroups per CU, two waves per SIMD.
template <bool UKS, bool RUN>
__global__ void __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(2)))
fwd_int8_b128_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                     const int8_t* __restrict__ qi, const float* __restrict__ qs,
                     const int8_t* __restrict__ ki, const float* __restrict__ ks,
                     const int8_t* __restrict__ vi, const float* __restrict__ vscale,
                     int64_t TP, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                     int64_t npad, const int32_t* __restrict__ counts,
                     const uint32_t* __restrict__ mask, int T,
                     int H, int NT, int W, float c, uint16_t* __restrict__ o, int64_t so_b,
                     int64_t so_t, int64_t so_h, int kst, int64_t ksh) {
  constexpr int BLK = 128, NTHREADS = 256;
  __shared__ __align__(256) char arena[2 * kBlkKStride + 2 * kBlkVStride];
  __shared__ TileList tl;
  const auto Kp = [&](int i) { return arena + i * kBlkKStride; };
  const auto Vp = [&](int i) { return arena + 2 * kBlkKStride + i * kBlkVStride; };

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  int bh, qb;
  tile_coords_lpt<kLptTokens / BLK>(counts, NT, bh, qb);
  const int b = bh / H, h = bh % H;
  const int64_t row = static_cast<int64_t>(bh) * NT + qb;

  const int ntiles = build_tile_list<BLK>(tl, mask, row, NT, W, T);
  if (ntiles == 0) return;  // cannot happen for routed masks: the diagonal is exact
  const int nexact = tl.nexact;  // exact 64-key tiles, list order
  // full exact blocks: list entries [0, nfb); a ragged last block (T not a
  // multiple of 128) keeps its tiles [2 nfb, nexact) for the plain path
  const int nfb = tl.nblk - ((tl.last == NT - 1 && (T % BLK) != 0) ? 1 : 0);

  const int64_t bhD = (static_cast<int64_t>(b) * npad * H + h) * kD;
  const KVSource src{nullptr, 0, nullptr, 0, kc + bhD, static_cast<int64_t>(H) * kD, vc + bhD};
  const I8Source is{ki + (static_cast<int64_t>(b) * TP * H + h) * kD,
                    ks + static_cast<int64_t>(b) * TP * H + h * ksh,
                    vi + (static_cast<int64_t>(b) * TP * H + h) * kD,
                    static_cast<int64_t>(H) * kD, kst};
  I8Offsets<NTHREADS> ioff;
  ioff.init(is.srow, kst);
  const uint32_t ks_blk = static_cast<uint32_t>((32 * wave + lane) * kst * 4);
  const uint32_t kb = lds_addr(arena);
  const auto kbuf_at = [&](int i) { return kb + i * kBlkKStride; };
  const auto vbuf_at = [&](int i) { return kb + 2 * kBlkKStride + i * kBlkVStride; };
  const auto blk_first = [&](int e) { return __builtin_amdgcn_readfirstlane(blist_lds()[e] * BLK); };
  const auto issue_k = [&](int e, int i) { issue_blk<true>(kbuf_at(i), is.ki, is, blk_first(e), ioff.k, ks_blk); };
  const auto issue_v = [&](int e, int i) { issue_blk<false>(vbuf_at(i), is.vi, is, blk_first(e), ioff.v, 0u); };

  if (nfb > 0) {
    issue_k(0, 0);
    issue_v(0, 0);
    if (nfb > 1) issue_k(1, 1);
  }
  const int qrow = qb * BLK + wave * 32 + col;
  const bool qvalid = qrow < T;
  SoftmaxState st;
  st.init();

  // ---- exact blocks and tiles (int8 Q: 16 VGPRs)
  if (nexact > 0) {
    i32x4 qireg[4];
    float qsl = 0.f;
    {
      const int64_t qoff = (static_cast<int64_t>(b) * TP + qrow) * H + h;
      const int8_t* qip = qi + qoff * kD + half * 16;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc) {
        uint4 r = make_uint4(0u, 0u, 0u, 0u);
        if (qvalid) r = *reinterpret_cast<const uint4*>(qip + cc * 32);
        qireg[cc] = __builtin_bit_cast(i32x4, r);
      }
      if (qvalid) qsl = qs[qoff] * c;
    }
    if (nfb > 0) {
      f32x16 sa[4], sb[4];
      float fa, fb;  // the score factors of sa, sb
      wait_tile_copies();
      __syncthreads();
      {
        i32x16 si[4];
#pragma unroll
        for (int m = 0; m < 4; ++m) si[m] = qk_chunk(Kp(0), qireg, m, col, half);
        scale_block<UKS>(Kp(0), si, half, sa);
        fa = tile_qsl<UKS>(Kp(0), kBlkKsOffset, qsl);
      }
      __syncthreads();  // K(0) is refilled (K of block 2) by the first step
      int e = 0;
      // Step e needs e + 1 < nfb; K(e+2) past the last block is clamped to it
      // (a redundant copy into a buffer nothing reads afterwards).
      const auto step = [&](const f32x16 (&sc)[4], float fc, f32x16 (&sn)[4], float& fn) {
        issue_k(min(e + 2, nfb - 1), e & 1);
        issue_v(e + 1, (e + 1) & 1);
        block_step<true, UKS, RUN>(st, sc, sn, Kp((e + 1) & 1), Vp(e & 1), qireg, fc, lane);
        fn = tile_qsl<UKS>(Kp((e + 1) & 1), kBlkKsOffset, qsl);
        wait_tile_copies();
        __syncthreads();
        ++e;
      };
      while (e + 2 < nfb) {
        step(sa, fa, sb, fb);
        step(sb, fb, sa, fa);
      }
      f32x16 dummy[4];
      if (e + 1 < nfb) {
        step(sa, fa, sb, fb);
        block_step<false, UKS, RUN>(st, sb, dummy, nullptr, Vp(e & 1), qireg, fb, lane);
      } else {
        block_step<false, UKS, RUN>(st, sa, dummy, nullptr, Vp(e & 1), qireg, fa, lane);
      }
      __syncthreads();
    }
    // tiles of a ragged last block: plain, masked, one at a time
    for (int t = 2 * nfb; t < nexact; ++t) {
      const TileDesc td = exact_desc<BLK>(tl, t, T, NT);
      issue_i8<NTHREADS, false, true>(kbuf_at(0), is.ki, is, td.first, td.nvalid, 0, 0, false);
      issue_i8<NTHREADS, false, false>(vbuf_at(0), is.vi, is, td.first, td.nvalid, 0, 0, true);
      wait_tile_copies();
      __syncthreads();
      i32x16 si[2];
      f32x16 s[2];
      const char* kt = Kp(0);
      qk_i8_tile(kt, qireg, col, half, si);
      scale_scores<UKS>(kt, si, half, s);
#pragma unroll
      for (int m = 0; m < 2; ++m) {
        const uint32_t bits = static_cast<uint32_t>(td.amask >> (32 * m + 4 * half));
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s[m][r] = ((bits >> (8 * (r >> 2) + (r & 3))) & 1u) ? s[m][r] : -INFINITY;
      }
      exact_softmax_pv<true, RUN>(st, s, Vp(0), tile_qsl<UKS>(kt, kKsOffset, qsl), lane);
      __syncthreads();
    }
    // The per-channel V scale, common to every exact block; the empty asm
    // keeps its 64 loads here.
    const float* vsc = vscale + static_cast<int64_t>(bh) * kD;
    asm volatile("" : "+s"(vsc));
    if constexpr (RUN) {
      run_finish(st, vsc, half);
    } else {
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.acc[dt][r] *= vsc[32 * dt + 8 * (r >> 2) + 4 * half + (r & 3)];
    }
  }

  // ---- pooled tiles (bf16 Q: 32 VGPRs), double buffered
  if (nexact < ntiles) {
    bf16x8 qreg[8];
    const uint16_t* qp = q + b * sq_b + static_cast<int64_t>(qrow) * sq_t + h * sq_h + half * 8;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      uint4 r = make_uint4(0u, 0u, 0u, 0u);
      if (qvalid) r = *reinterpret_cast<const uint4*>(qp + cc * 16);
      qreg[cc] = __builtin_bit_cast(bf16x8, r);
    }
    const auto issue_pooled = [&](int p, int i) {
      const TileDesc td = pooled_desc(tl, p, NT);
      issue_generic<NTHREADS>(kbuf_at(i), 0, td, src);
      issue_generic<NTHREADS>(vbuf_at(i), 1, td, src);
    };
    const int npool = ntiles - nexact;
    issue_pooled(0, 0);  // every earlier copy has landed
    for (int p = 0; p < npool; ++p) {
      wait_tile_copies();  // pooled tile p: the only copies in flight
      __syncthreads();
      if (p + 1 < npool) issue_pooled(p + 1, (p + 1) & 1);
      f32x16 s[2];
      qk_tile(reinterpret_cast<const uint16_t*>(Kp(p & 1)), qreg, col, half, s);
      finish_tile<BLK>(st, s, reinterpret_cast<const uint16_t*>(Vp(p & 1)), pooled_desc(tl, p, NT), c,
                       lane, NT, T);
      __syncthreads();
    }
  }
  wait_tile_copies();
  store_rows(st, o + b * so_b + h * so_h, so_t, qrow, T, half);
}

template <int BLK, bool PV, bool UKS, bool RUN>
void launch_i8(uint32_t grid, hipStream_t s, const uint16_t* q, int64_t sq_b, int64_t sq_t,
               int64_t sq_h, const int8_t* qi, const float* qs, const int8_t* ki, const float* ks,
               const int8_t* vi, const float* vscale, const uint16_t* v, int64_t sv_b,
               int64_t sv_t, int64_t sv_h, int64_t TP, const uint16_t* kc, const uint16_t* vc,
               int64_t npad, const int32_t* counts, const uint32_t* mask,
               int T, int H, int NT, int W, float c, uint16_t* o, int64_t so_b, int64_t so_t,
               int64_t so_h, int kst, int64_t ksh) {
  hipLaunchKernelGGL((fwd_int8_kernel<BLK, PV, UKS, RUN>), dim3(grid), dim3(BLK * 2), blist_lds_bytes(NT), s, q, sq_b, sq_t,
                     sq_h, qi, qs, ki, ks, vi, vscale, v, sv_b, sv_t, sv_h, TP, kc, vc, npad,
                     counts, mask, T, H, NT, W, c, o, so_b, so_t, so_h, kst, ksh);
}

template <int BLK, bool PV, bool RUN = false>
void launch_i8_ks(bool uks, uint32_t grid, hipStream_t s, const uint16_t* q, int64_t sq_b,
                  int64_t sq_t, int64_t sq_h, const int8_t* qi, const float* qs, const int8_t* ki,
                  const float* ks, const int8_t* vi, const float* vscale, const uint16_t* v,
                  int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t TP, const uint16_t* kc,
                  const uint16_t* vc, int64_t npad, const int32_t* counts, const uint32_t* mask, int T, int H, int NT, int W, float c, uint16_t* o,
                  int64_t so_b, int64_t so_t, int64_t so_h, int kst, int64_t ksh) {
  (uks ? launch_i8<BLK, PV, true, RUN> : launch_i8<BLK, PV, false, RUN>)(
      grid, s, q, sq_b, sq_t, sq_h, qi, qs, ki, ks, vi, vscale, v, sv_b, sv_t, sv_h, TP, kc, vc,
      npad, counts, mask, T, H, NT, W, c, o, so_b, so_t, so_h, kst, ksh);
}

}  // namespace int8fwd

int fwd_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const int8_t* qi,
             const float* qs, const int8_t* ki, const float* ks, const int8_t* vi,
             const float* vscale, const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
             int64_t TP, const uint16_t* kc, const uint16_t* vc, int64_t npad,
             const int32_t* counts, const uint32_t* mask, int64_t B,
             int64_t T, int64_t H, int64_t D, int64_t block, float scale, int int8_pv,
             uint16_t* o, int64_t so_b, int64_t so_t, int64_t so_h, solattn_stream_t stream,
             bool uniform_ks, bool ks_head_major) {
  if (int rc = check_fwd_common(q, sq_b, sq_t, sq_h, kc, vc, npad, counts, mask, B, T, H, D,
                                block, o, so_b, so_t, so_h, "fwd_int8"))
    return rc;
  SOLATTN_REQUIRE(TP >= T, SOLATTN_EINVAL, "fwd_int8: TP < T");
  SOLATTN_REQUIRE(int8_pv >= SOLATTN_PV_BF16 && int8_pv <= SOLATTN_PV_INT8_RUNNING, SOLATTN_EINVAL,
                  "fwd_int8: int8_pv %d is not a SOLATTN_PV_* mode", int8_pv);
  SOLATTN_REQUIRE(qi && qs && ki && ks, SOLATTN_EINVAL, "fwd_int8: null int8 operand");
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(qi) % 16 == 0 && reinterpret_cast<uintptr_t>(ki) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(ks) % 4 == 0,
                  SOLATTN_EINVAL, "fwd_int8: qi/ki must be 16-byte aligned");
  // Lane offsets within a 64-row int8 tile are kept in 32 bits.
  SOLATTN_REQUIRE(H * D < (1ll << 24), SOLATTN_EUNSUPPORTED, "fwd_int8: H*D beyond 2^24");
  if (int8_pv) {
    SOLATTN_REQUIRE(vi && vscale && reinterpret_cast<uintptr_t>(vi) % 16 == 0, SOLATTN_EINVAL,
                    "fwd_int8: int8_pv needs 16-byte aligned vi and vscale");
  } else {
    SOLATTN_REQUIRE(v && reinterpret_cast<uintptr_t>(v) % 16 == 0 && sv_b % 8 == 0 &&
                        sv_t % 8 == 0 && sv_h % 8 == 0 && sv_t >= 0 && sv_t < (1ll << 24),
                    SOLATTN_EINVAL, "fwd_int8: bf16 v must be 16-byte aligned with strides multiple of 8");
  }
  const int64_t NT = cdiv(T, block);
  const int W = static_cast<int>(cdiv(NT, 32));
  const float c = scale * kLog2e;
  const uint32_t grid = static_cast<uint32_t>(B * H * NT);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  // ks: token-major [B, TP, H] (the reference's) or head-major [B, H, TP]
  const int kst = ks_head_major ? 1 : static_cast<int>(H);
  const int64_t ksh = ks_head_major ? TP : 1;
#define SOLATTN_I8_ARGS                                                                          \
  grid, s, q, sq_b, sq_t, sq_h, qi, qs, ki, ks, vi, vscale, v, sv_b, sv_t, sv_h, TP, kc, vc, npad, \
      counts, mask, static_cast<int>(T), static_cast<int>(H), static_cast<int>(NT), W, c, o, \
      so_b, so_t, so_h, kst, ksh
  const bool run = int8_pv == SOLATTN_PV_INT8_RUNNING;
  if (block == 128) {
    if (int8_pv) {
      const auto kern = uniform_ks ? (run ? int8fwd::fwd_int8_b128_kernel<true, true>
                                          : int8fwd::fwd_int8_b128_kernel<true, false>)
                                   : (run ? int8fwd::fwd_int8_b128_kernel<false, true>
                                          : int8fwd::fwd_int8_b128_kernel<false, false>);
      hipLaunchKernelGGL(kern, dim3(grid), dim3(256), blist_lds_bytes(NT), s, q, sq_b, sq_t, sq_h,
                         qi, qs, ki, ks, vi, vscale, TP, kc, vc, npad, counts, mask,
                         static_cast<int>(T), static_cast<int>(H), static_cast<int>(NT), W, c, o,
                         so_b, so_t, so_h, kst, ksh);
    } else {
      int8fwd::launch_i8_ks<128, false>(uniform_ks, SOLATTN_I8_ARGS);
    }
  } else {
    if (run) int8fwd::launch_i8_ks<64, true, true>(uniform_ks, SOLATTN_I8_ARGS);
    else if (int8_pv) int8fwd::launch_i8_ks<64, true>(uniform_ks, SOLATTN_I8_ARGS);
    else int8fwd::launch_i8_ks<64, false>(uniform_ks, SOLATTN_I8_ARGS);
  }
#undef SOLATTN_I8_ARGS
  return check_launch("fwd_int8");
}

}  // namespace solattn

extern "C" int solattn_fwd_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                const int8_t* qi, const float* qs, const int8_t* ki,
                                const float* ks, const int8_t* vi, const float* vscale,
                                const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                int64_t TP, const uint16_t* kc, const uint16_t* vc, int64_t npad,
                                const int32_t* counts, const uint32_t* mask,
                                int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                                float scale, int int8_pv, uint16_t* o, int64_t so_b, int64_t so_t,
                                int64_t so_h, solattn_stream_t stream) {
  solattn::clear_error();
  return solattn::fwd_int8(q, sq_b, sq_t, sq_h, qi, qs, ki, ks, vi, vscale, v, sv_b, sv_t, sv_h,
                           TP, kc, vc, npad, counts, mask, B, T, H, D, block, scale,
                           int8_pv, o, so_b, so_t, so_h, stream, false);
}
