// INT8 Sol-Attn forward on gfx950 MFMA (/root/reference/_int8_fwd.py:208-372).
//
// Exact tiles: S = int32(qi . ki) * ((qs * c) * ks) on v_mfma_i32_32x32x32_i8.
//   INT8_PV: P is quantised per row against the tile's own max,
//     pe = exp2(s - bmax), code = min(pe*127 + 0.5, 127), and multiplied with
//     per-channel int8 V on the i8 MFMA; the row factor beta/127 (beta =
//     exp2(bmax - m)) is applied per tile, the channel scale vscale[d] once at
//     the end of the exact phase (it is the same for every tile).
//   otherwise: P.V in bf16 against the bf16 V, as in the BF16 forward.
// Pooled tiles run afterwards in bf16 on the centred kc and vc. Tile order is
// free: the online softmax is exact under reordering, up to fp32 rounding.
//
// Tiles are copied global -> LDS directly (double buffered). int8 K and V stay
// row-major (128-byte rows, XOR-swizzled 16-byte chunks); ds_read_b64_tr_b8
// delivers V transposed as the MFMA A operand.
#include "common.hpp"
#include "fwd_common.hpp"

namespace solattn {

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

struct I8Source {
  const int8_t* ki;  // rows of this batch/head, stride srow bytes
  const float* ks;   // stride H floats
  const int8_t* vi;
  const uint16_t* v;  // bf16 V (INT8_PV off)
  int64_t sv;
  int64_t srow;
  int H;
};

// Tile n: the exact tiles first (n < nexact), then the pooled tiles.
template <int BLK>
__device__ __forceinline__ TileDesc tile_desc_i8(const TileList& tl, int n, int T, int NT) {
  return n < tl.nexact ? tile_desc<BLK>(tl, n + tl.npool, T, NT) : tile_desc<BLK>(tl, n - tl.nexact, T, NT);
}

template <int BLK, int NTHREADS, bool INT8_PV>
__device__ __forceinline__ void issue_i8(uint16_t* kdst, uint16_t* vdst, const TileList& tl, int n,
                                         const KVSource& src, const I8Source& is,
                                         const TileOffsets<NTHREADS>& off, int T, int NT) {
  if (n >= tl.nexact) {
    issue_half<BLK, NTHREADS>(kdst, 0, tl, n - tl.nexact, src, off, T, NT);
    issue_half<BLK, NTHREADS>(vdst, 1, tl, n - tl.nexact, src, off, T, NT);
    return;
  }
  const TileDesc td = tile_desc_i8<BLK>(tl, n, T, NT);
  const int wave_base = threadIdx.x & ~63;
  char* kb = reinterpret_cast<char*>(kdst);
  char* vb = reinterpret_cast<char*>(vdst);
  // ks[64] (stride H floats) by 4-byte copies, behind the int8 rows.
  if (threadIdx.x < kKeys) {
    const int row = static_cast<int>(threadIdx.x) < td.nvalid ? static_cast<int>(threadIdx.x) : 0;
    g2l4(is.ks + static_cast<int64_t>(td.first + row) * is.H, kb + kKsOffset);
  }
#pragma unroll
  for (int u = 0; u < kKeys * 8 / NTHREADS; ++u) {
    const int e = threadIdx.x + NTHREADS * u;
    const int row = e >> 3, pc = e & 7;
    const int64_t srow = td.first + (row < td.nvalid ? row : 0);
    const int lds = (wave_base + NTHREADS * u) * 16;
    g2l16(is.ki + srow * is.srow + swz_ki(row, pc) * 16, kb + lds);
    if constexpr (INT8_PV) g2l16(is.vi + srow * is.srow + swz_vi(row, pc) * 16, vb + lds);
  }
  if constexpr (!INT8_PV) issue_half<BLK, NTHREADS>(vdst, 1, tl, n + tl.npool, src, off, T, NT);
}

__device__ __forceinline__ uint32_t quant_p4(float a, float b, float c, float d) {
  // min(pe*127 + 0.5, 127) truncated: pe is in [0, 1]
  const uint32_t qa = static_cast<uint32_t>(fminf(fmaf(a, 127.f, 0.5f), 127.f));
  const uint32_t qb = static_cast<uint32_t>(fminf(fmaf(b, 127.f, 0.5f), 127.f));
  const uint32_t qc = static_cast<uint32_t>(fminf(fmaf(c, 127.f, 0.5f), 127.f));
  const uint32_t qd = static_cast<uint32_t>(fminf(fmaf(d, 127.f, 0.5f), 127.f));
  return qa | (qb << 8) | (qc << 16) | (qd << 24);
}

__device__ __forceinline__ i32x2 tr8(const char* p) {
  typedef int v2i32 __attribute__((ext_vector_type(2)));
  const v2i32 r = __builtin_amdgcn_ds_read_tr8_b64_v2i32((__attribute__((address_space(3))) v2i32*)(p));
  return __builtin_bit_cast(i32x2, r);
}

// One exact int8 tile: S^T = Ki . Qi^T, online softmax, P.V.
template <bool INT8_PV>
__device__ __forceinline__ void exact_i8(SoftmaxState& st, const uint16_t* kt16, const uint16_t* vt16,
                                         const i32x4 (&qireg)[4], float qsl, const TileDesc& td,
                                         int lane) {
  const int col = lane & 31, half = lane >> 5;
  const char* kt = reinterpret_cast<const char*>(kt16);
  i32x16 si[2];
  const i32x16 zero = {};
#pragma unroll
  for (int cc = 0; cc < 4; ++cc)
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = 32 * m + col;
      const i32x4 a = *reinterpret_cast<const i32x4*>(kt + row * kI8Row + swz_ki(row, 2 * cc + half) * 16);
      si[m] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qireg[cc], cc == 0 ? zero : si[m], 0, 0, 0);
    }
  // s = int32 * (qs*c * ks): the reference's exact_scores (/root/reference/_int8_fwd.py:328-330).
  const float* ksl = reinterpret_cast<const float*>(kt + kKsOffset);
  f32x16 s[2];
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < 2; ++m) {
    const uint32_t bits = static_cast<uint32_t>(td.amask >> (32 * m + 4 * half));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float4 k4 = *reinterpret_cast<const float4*>(ksl + 32 * m + 8 * i + 4 * half);
      const float kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float v = static_cast<float>(si[m][4 * i + j]) * (qsl * kk[j]);
        s[m][4 * i + j] = ((bits >> (8 * i + j)) & 1u) ? v : -INFINITY;
        mx = fmaxf(mx, s[m][4 * i + j]);
      }
    }
  }
  const float bmax = fmaxf(mx, __shfl_xor(mx, 32));
  const float m_new = bmax > st.m + kMaxSlack ? bmax : st.m;
  const float alpha = st.m == m_new ? 1.f : __builtin_amdgcn_exp2f(st.m - m_new);
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[dt][r] *= alpha;
  }
  if constexpr (INT8_PV) {
    // P against the tile max: pe in [0, 1], beta carries it to the running max
    // (/root/reference/_int8_fwd.py:348-353).
    const float beta = __builtin_amdgcn_exp2f(bmax - m_new);
    float psum = 0.f;
    i32x4 pb[2];
#pragma unroll
    for (int m = 0; m < 2; ++m) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[m][r] = __builtin_amdgcn_exp2f(s[m][r] - bmax);
        psum += s[m][r];
      }
#pragma unroll
      for (int w = 0; w < 4; ++w)
        pb[m][w] = static_cast<int>(quant_p4(s[m][4 * w], s[m][4 * w + 1], s[m][4 * w + 2], s[m][4 * w + 3]));
    }
    st.l = fmaf(st.l, alpha, beta * psum);
    const float f = beta * (1.f / 127.f);
    // O^T += Vi^T . Pi^T: lane (channel 32dt + col, half) takes keys
    // 32ks + 8i + 4*half + j (i, j < 4) from two ds_read_tr8: within a 16-lane
    // group, lane s supplies key (s >> 1) of the 8 keys, channels 8*(s & 1)..+7.
    const char* vt = reinterpret_cast<const char*>(vt16);
    const int g = lane >> 4, sl = lane & 15;
    const int kk = sl >> 1;                       // key index within the 8 read
    const int key_in = 8 * (kk >> 2) + 4 * half + (kk & 3);
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int chunk = 2 * dt + (g & 1);         // 16-byte chunk of channels 32dt + 16(g&1)
      i32x16 pv;
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        const int r0 = 32 * ks + key_in, r1 = r0 + 16;
        const i32x2 lo = tr8(vt + r0 * kI8Row + swz_vi(r0, chunk) * 16 + 8 * (sl & 1));
        const i32x2 hi = tr8(vt + r1 * kI8Row + swz_vi(r1, chunk) * 16 + 8 * (sl & 1));
        const i32x4 a = {lo[0], lo[1], hi[0], hi[1]};
        pv = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, pb[ks], ks == 0 ? zero : pv, 0, 0, 0);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[dt][r] = fmaf(static_cast<float>(pv[r]), f, st.acc[dt][r]);
    }
  } else {
    float psum = 0.f;
    const float neg = -m_new;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[m][r] = __builtin_amdgcn_exp2f(s[m][r] + neg);
        psum += s[m][r];
      }
    st.l = fmaf(st.l, alpha, psum);
    pv_tr16(vt16, s, lane, st.acc);
  }
  st.m = m_new;
}

template <int BLK, bool INT8_PV>
__global__ void __launch_bounds__(BLK * 2, 2)
fwd_int8_kernel(const uint16_t* __restrict__ q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                const int8_t* __restrict__ qi, const float* __restrict__ qs,
                const int8_t* __restrict__ ki, const float* __restrict__ ks,
                const int8_t* __restrict__ vi, const float* __restrict__ vscale,
                const uint16_t* __restrict__ v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                int64_t TP, const uint16_t* __restrict__ kc, const uint16_t* __restrict__ vc,
                int64_t npad, const int32_t* __restrict__ counts, const int16_t* __restrict__ lists,
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
  const int nexact = tl.nexact;

  const int64_t bhD = (static_cast<int64_t>(b) * npad * H + h) * kD;
  const KVSource src{nullptr, 0, INT8_PV ? nullptr : v + b * sv_b + h * sv_h, sv_t, kc + bhD,
                     static_cast<int64_t>(H) * kD, vc + bhD};
  const I8Source is{ki + (static_cast<int64_t>(b) * TP * H + h) * kD,
                    ks + static_cast<int64_t>(b) * TP * H + h,
                    INT8_PV ? vi + (static_cast<int64_t>(b) * TP * H + h) * kD : nullptr,
                    INT8_PV ? nullptr : v + b * sv_b + h * sv_h,
                    sv_t,
                    static_cast<int64_t>(H) * kD,
                    H};
  TileOffsets<NTHREADS> off;
  off.init(0, sv_t);
  issue_i8<BLK, NTHREADS, INT8_PV>(kbuf[0], vbuf[0], tl, 0, src, is, off, T, NT);

  const int qrow = qb * BLK + wave * 32 + col;
  const bool qvalid = qrow < T;
  SoftmaxState st;
  st.init();
  int n = 0;
  if (nexact > 0) {
    // Exact phase: int8 Q (16 VGPRs) only.
    i32x4 qireg[4];
    float qsl = 0.f;
    const int64_t qoff = (static_cast<int64_t>(b) * TP + qrow) * H + h;
    const int8_t* qip = qi + qoff * kD + half * 16;
#pragma unroll
    for (int cc = 0; cc < 4; ++cc) {
      uint4 r = make_uint4(0u, 0u, 0u, 0u);
      if (qvalid) r = *reinterpret_cast<const uint4*>(qip + cc * 32);
      qireg[cc] = __builtin_bit_cast(i32x4, r);
    }
    if (qvalid) qsl = qs[qoff] * c;
    wait_tile_copies();
    __syncthreads();
    for (; n < nexact; ++n) {
      if (n + 1 < ntiles)
        issue_i8<BLK, NTHREADS, INT8_PV>(kbuf[(n + 1) & 1], vbuf[(n + 1) & 1], tl, n + 1, src, is,
                                         off, T, NT);
      const TileDesc td = tile_desc_i8<BLK>(tl, n, T, NT);
      exact_i8<INT8_PV>(st, kbuf[n & 1], vbuf[n & 1], qireg, qsl, td, lane);
      wait_tile_copies();
      __syncthreads();
    }
    if constexpr (INT8_PV) {
      // Exact phase done: the per-channel V scale is the same for every tile.
      const float* vsc = vscale + static_cast<int64_t>(bh) * kD;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 16; ++r) st.acc[dt][r] *= vsc[32 * dt + 8 * (r >> 2) + 4 * half + (r & 3)];
    }
  }
  if (n < ntiles) {
    // Pooled phase: bf16 Q against the centred kc / vc.
    bf16x8 qreg[8];
    const uint16_t* qp = q + b * sq_b + static_cast<int64_t>(qrow) * sq_t + h * sq_h + half * 8;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      uint4 r = make_uint4(0u, 0u, 0u, 0u);
      if (qvalid) r = *reinterpret_cast<const uint4*>(qp + cc * 16);
      qreg[cc] = __builtin_bit_cast(bf16x8, r);
    }
    if (n == 0) {
      wait_tile_copies();
      __syncthreads();
    }
    for (; n < ntiles; ++n) {
      if (n + 1 < ntiles)
        issue_i8<BLK, NTHREADS, INT8_PV>(kbuf[(n + 1) & 1], vbuf[(n + 1) & 1], tl, n + 1, src, is,
                                         off, T, NT);
      const TileDesc td = tile_desc_i8<BLK>(tl, n, T, NT);
      f32x16 s[2];
      qk_swz(kbuf[n & 1], qreg, col, half, s);
      softmax_update<BLK>(st, s, td, c, half, NT, T);
      pv_tr16(vbuf[n & 1], s, lane, st.acc);
      wait_tile_copies();
      __syncthreads();
    }
  }

  store_output(st, o + b * so_b + h * so_h, so_t, qrow, T, half);
}

template <int BLK, bool PV>
void launch_i8(uint32_t grid, hipStream_t s, const uint16_t* q, int64_t sq_b, int64_t sq_t,
               int64_t sq_h, const int8_t* qi, const float* qs, const int8_t* ki, const float* ks,
               const int8_t* vi, const float* vscale, const uint16_t* v, int64_t sv_b,
               int64_t sv_t, int64_t sv_h, int64_t TP, const uint16_t* kc, const uint16_t* vc,
               int64_t npad, const int32_t* counts, const int16_t* lists, const uint32_t* mask,
               int T, int H, int NT, int W, float c, uint16_t* o, int64_t so_b, int64_t so_t,
               int64_t so_h) {
  hipLaunchKernelGGL((fwd_int8_kernel<BLK, PV>), dim3(grid), dim3(BLK * 2), 0, s, q, sq_b, sq_t,
                     sq_h, qi, qs, ki, ks, vi, vscale, v, sv_b, sv_t, sv_h, TP, kc, vc, npad,
                     counts, lists, mask, T, H, NT, W, c, o, so_b, so_t, so_h);
}

}  // namespace solattn

using namespace solattn;

extern "C" int solattn_fwd_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                const int8_t* qi, const float* qs, const int8_t* ki,
                                const float* ks, const int8_t* vi, const float* vscale,
                                const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                int64_t TP, const uint16_t* kc, const uint16_t* vc, int64_t npad,
                                const int32_t* counts, const int16_t* lists, const uint32_t* mask,
                                int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                                float scale, int int8_pv, uint16_t* o, int64_t so_b, int64_t so_t,
                                int64_t so_h, solattn_stream_t stream) {
  clear_error();
  if (int rc = check_fwd_common(q, sq_b, sq_t, sq_h, kc, vc, npad, counts, lists, mask, B, T, H, D,
                                block, o, so_b, so_t, so_h, "fwd_int8"))
    return rc;
  SOLATTN_REQUIRE(TP >= T, SOLATTN_EINVAL, "fwd_int8: TP < T");
  SOLATTN_REQUIRE(qi && qs && ki && ks, SOLATTN_EINVAL, "fwd_int8: null int8 operand");
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(qi) % 16 == 0 && reinterpret_cast<uintptr_t>(ki) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(ks) % 4 == 0,
                  SOLATTN_EINVAL, "fwd_int8: qi/ki must be 16-byte aligned");
  if (int8_pv) {
    SOLATTN_REQUIRE(vi && vscale && reinterpret_cast<uintptr_t>(vi) % 16 == 0, SOLATTN_EINVAL,
                    "fwd_int8: int8_pv needs 16-byte aligned vi and vscale");
  } else {
    SOLATTN_REQUIRE(v && reinterpret_cast<uintptr_t>(v) % 16 == 0 && sv_b % 8 == 0 &&
                        sv_t % 8 == 0 && sv_h % 8 == 0 && sv_t < (1ll << 24),
                    SOLATTN_EINVAL, "fwd_int8: bf16 v must be 16-byte aligned with strides multiple of 8");
  }
  const int64_t NT = cdiv(T, block);
  const int W = static_cast<int>(cdiv(NT, 32));
  const float c = scale * kLog2e;
  const uint32_t grid = static_cast<uint32_t>(B * H * NT);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
#define SOLATTN_I8_ARGS                                                                          \
  grid, s, q, sq_b, sq_t, sq_h, qi, qs, ki, ks, vi, vscale, v, sv_b, sv_t, sv_h, TP, kc, vc, npad, \
      counts, lists, mask, static_cast<int>(T), static_cast<int>(H), static_cast<int>(NT), W, c, o, \
      so_b, so_t, so_h
  if (block == 128) {
    if (int8_pv) launch_i8<128, true>(SOLATTN_I8_ARGS);
    else launch_i8<128, false>(SOLATTN_I8_ARGS);
  } else {
    if (int8_pv) launch_i8<64, true>(SOLATTN_I8_ARGS);
    else launch_i8<64, false>(SOLATTN_I8_ARGS);
  }
#undef SOLATTN_I8_ARGS
  return check_launch("fwd_int8");
}
