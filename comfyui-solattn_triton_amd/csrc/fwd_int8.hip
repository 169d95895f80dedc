// INT8 Sol-Attn forward on gfx950 MFMA (/root/reference/_int8_fwd.py:208-372).
//
// Exact tiles: S = int32(qi . ki) * ((qs * c) * ks) with v_mfma_i32_32x32x32_i8.
//   INT8_PV: P is quantised per row against the tile's own max,
//     pe = exp2(s - bmax), code = min(pe*127 + 0.5, 127), and multiplied with
//     per-channel int8 V on the i8 MFMA; the row factor beta/127 (beta =
//     exp2(bmax - m)) is applied per tile, the channel scale vscale[d] once at
//     the end of the exact phase (it is the same for every tile).
//   otherwise: P.V in bf16 against the bf16 V, as in the BF16 forward.
// Pooled tiles run afterwards in bf16 on the centred kc and vc.
// Order of the tiles is free: the online softmax is exact under reordering,
// up to fp32 rounding.
#include "common.hpp"
#include "fwd_common.hpp"

namespace solattn {

constexpr int kKI8Stride = kD + 16;     // bytes per int8 K row in LDS (144)
constexpr int kVI8Stride = kKeys + 16;  // bytes per int8 V^T row in LDS (80)
constexpr int kKsOffset = kKeys * kKI8Stride;  // ks[64] after the int8 K rows

__device__ __forceinline__ int8_t* k_i8(TileBuf& b) { return reinterpret_cast<int8_t*>(b.k); }
__device__ __forceinline__ const int8_t* k_i8(const TileBuf& b) {
  return reinterpret_cast<const int8_t*>(b.k);
}
__device__ __forceinline__ float* ks_f(TileBuf& b) {
  return reinterpret_cast<float*>(reinterpret_cast<char*>(b.k) + kKsOffset);
}
__device__ __forceinline__ const float* ks_f(const TileBuf& b) {
  return reinterpret_cast<const float*>(reinterpret_cast<const char*>(b.k) + kKsOffset);
}
__device__ __forceinline__ int8_t* vt_i8(TileBuf& b) { return reinterpret_cast<int8_t*>(b.vt); }
__device__ __forceinline__ const int8_t* vt_i8(const TileBuf& b) {
  return reinterpret_cast<const int8_t*>(b.vt);
}

struct I8Source {
  const int8_t* ki;  // [T][H*D] rows of this batch/head
  const float* ks;   // stride H
  const int8_t* vi;
  const uint16_t* v;  // bf16 V (INT8_PV off)
  int64_t sv;
  int64_t srow;  // row stride of ki/vi (H*D) and ks (H)
  int H;
};

// INT8 tiles first (n < nexact), then pooled tiles.
template <int BLK>
__device__ __forceinline__ TileDesc tile_desc_i8(const TileList& sh, int n, int T, int NT) {
  if (n < sh.nexact) {
    // tile_desc() numbers exact tiles after the pooled ones
    return tile_desc<BLK>(sh, n + sh.npool, T, NT);
  }
  return tile_desc<BLK>(sh, n - sh.nexact, T, NT);
}

template <int BLK, int NTHREADS, bool INT8_PV>
__device__ __forceinline__ void load_tile_i8(TileRegs<NTHREADS>& r, float& ksr,
                                             const TileList& sh, int n, const KVSource& src,
                                             const I8Source& is, int T, int NT) {
  const TileDesc td = tile_desc_i8<BLK>(sh, n, T, NT);
  if (td.pooled) {
    load_tile<BLK, NTHREADS>(r, sh, n - sh.nexact, src, T, NT);
    return;
  }
  const uint4 z = make_uint4(0u, 0u, 0u, 0u);
  // int8 K: 64 rows x 8 chunks of 16 bytes.
  constexpr int KCH = kKeys * kD / 16 / NTHREADS;
#pragma unroll
  for (int u = 0; u < KCH; ++u) {
    const int e = threadIdx.x + NTHREADS * u;
    const int row = e >> 3, cc = e & 7;
    r.k[u] = row < td.nvalid
                 ? *reinterpret_cast<const uint4*>(is.ki + static_cast<int64_t>(td.first + row) * is.srow + cc * 16)
                 : z;
  }
  ksr = 0.f;
  if (threadIdx.x < kKeys && static_cast<int>(threadIdx.x) < td.nvalid)
    ksr = is.ks[static_cast<int64_t>(td.first + threadIdx.x) * is.H];
  if constexpr (INT8_PV) {
    // int8 V: 16 key quads x 8 chunks of 16 channels, 4 rows each.
    constexpr int UNITS = kKeys / 4 * kD / 16;
    static_assert(UNITS <= NTHREADS, "one int8 V unit per thread at most");
    if (threadIdx.x < UNITS) {
      const int kq = threadIdx.x & 15, dc = threadIdx.x >> 4;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int row = 4 * kq + x;
        r.v[0][x] = row < td.nvalid
                        ? *reinterpret_cast<const uint4*>(is.vi + static_cast<int64_t>(td.first + row) * is.srow + dc * 16)
                        : z;
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < TileRegs<NTHREADS>::VU; ++u) {
      const int e = threadIdx.x + NTHREADS * u;
      const int kq = e & 15, dc = e >> 4;
#pragma unroll
      for (int x = 0; x < 4; ++x) {
        const int row = 4 * kq + x;
        r.v[u][x] = row < td.nvalid ? ld16(is.v + static_cast<int64_t>(td.first + row) * is.sv + dc * 8) : z;
      }
    }
  }
}

__device__ __forceinline__ uint32_t byte_of(const uint4& a, int i) {
  return (word_of(a, i >> 2) >> (8 * (i & 3))) & 0xffu;
}

template <int BLK, int NTHREADS, bool INT8_PV>
__device__ __forceinline__ void store_tile_i8(const TileRegs<NTHREADS>& r, float ksr, bool pooled,
                                              TileBuf& buf) {
  if (pooled) {
    store_tile<NTHREADS>(r, buf);
    return;
  }
  constexpr int KCH = kKeys * kD / 16 / NTHREADS;
#pragma unroll
  for (int u = 0; u < KCH; ++u) {
    const int e = threadIdx.x + NTHREADS * u;
    const int row = e >> 3, cc = e & 7;
    *reinterpret_cast<uint4*>(k_i8(buf) + row * kKI8Stride + cc * 16) = r.k[u];
  }
  if (threadIdx.x < kKeys) ks_f(buf)[threadIdx.x] = ksr;
  if constexpr (INT8_PV) {
    // V^T with keys permuted inside each group of 32 so that one lane's 16 keys
    // (8i + 4h + j) sit at 16h + 4i + j: one 16-byte read per MFMA operand.
    constexpr int UNITS = kKeys / 4 * kD / 16;
    if (threadIdx.x < UNITS) {
      const int kq = threadIdx.x & 15, dc = threadIdx.x >> 4;
      constexpr int u = 0;
      const int g = kq >> 3, i = (kq & 7) >> 1, hh = kq & 1;
      const int pos = 32 * g + 16 * hh + 4 * i;
#pragma unroll
      for (int el = 0; el < 16; ++el) {
        const uint32_t w = byte_of(r.v[u][0], el) | (byte_of(r.v[u][1], el) << 8) |
                           (byte_of(r.v[u][2], el) << 16) | (byte_of(r.v[u][3], el) << 24);
        *reinterpret_cast<uint32_t*>(vt_i8(buf) + (dc * 16 + el) * kVI8Stride + pos) = w;
      }
    }
  } else {
#pragma unroll
    for (int u = 0; u < TileRegs<NTHREADS>::VU; ++u) {
      const int e = threadIdx.x + NTHREADS * u;
      const int kq = e & 15, dc = e >> 4;
#pragma unroll
      for (int el = 0; el < 8; ++el) {
        const uint32_t a0 = word_of(r.v[u][0], el >> 1), a1 = word_of(r.v[u][1], el >> 1);
        const uint32_t a2 = word_of(r.v[u][2], el >> 1), a3 = word_of(r.v[u][3], el >> 1);
        uint2 p;
        if ((el & 1) == 0) {
          p.x = (a0 & 0xffffu) | (a1 << 16);
          p.y = (a2 & 0xffffu) | (a3 << 16);
        } else {
          p.x = (a0 >> 16) | (a1 & 0xffff0000u);
          p.y = (a2 >> 16) | (a3 & 0xffff0000u);
        }
        *reinterpret_cast<uint2*>(&buf.vt[(dc * 8 + el) * kVStride + 4 * kq]) = p;
      }
    }
  }
}

__device__ __forceinline__ uint32_t quant_p4(float a, float b, float c, float d) {
  // min(pe*127 + 0.5, 127) truncated: pe is in [0, 1]
  const uint32_t qa = static_cast<uint32_t>(fminf(fmaf(a, 127.f, 0.5f), 127.f));
  const uint32_t qb = static_cast<uint32_t>(fminf(fmaf(b, 127.f, 0.5f), 127.f));
  const uint32_t qc = static_cast<uint32_t>(fminf(fmaf(c, 127.f, 0.5f), 127.f));
  const uint32_t qd = static_cast<uint32_t>(fminf(fmaf(d, 127.f, 0.5f), 127.f));
  return qa | (qb << 8) | (qc << 16) | (qd << 24);
}

template <int BLK, bool INT8_PV>
__global__ void __launch_bounds__(BLK * 2)
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
  __shared__ TileBuf tbufs[2];
  __shared__ TileList sh;

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int col = lane & 31, half = lane >> 5;
  int bh, qb;
  tile_coords(blockIdx.x, gridDim.x, NT, bh, qb);
  const int b = bh / H, h = bh % H;
  const int64_t row = static_cast<int64_t>(bh) * NT + qb;

  const int ntiles = build_tile_list<BLK>(sh, counts, lists, mask, row, NT, W, T);
  if (ntiles == 0) return;  // cannot happen for routed lists: the diagonal is exact
  const int nexact = sh.nexact;

  const int qrow = qb * BLK + wave * 32 + col;
  const bool qvalid = qrow < T;
  bf16x8 qreg[8];
  i32x4 qireg[4];
  float qsl = 0.f;
  {
    const uint16_t* qp = q + b * sq_b + static_cast<int64_t>(qrow) * sq_t + h * sq_h + half * 8;
#pragma unroll
    for (int cc = 0; cc < 8; ++cc) {
      uint4 r = make_uint4(0u, 0u, 0u, 0u);
      if (qvalid) r = *reinterpret_cast<const uint4*>(qp + cc * 16);
      qreg[cc] = __builtin_bit_cast(bf16x8, r);
    }
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

  const int64_t bhD = (static_cast<int64_t>(b) * npad * H + h) * kD;
  const KVSource src{nullptr, 0, nullptr, 0, kc + bhD, static_cast<int64_t>(H) * kD, vc + bhD};
  const I8Source is{ki + (static_cast<int64_t>(b) * TP * H + h) * kD,
                    ks + static_cast<int64_t>(b) * TP * H + h,
                    INT8_PV ? vi + (static_cast<int64_t>(b) * TP * H + h) * kD : nullptr,
                    INT8_PV ? nullptr : v + b * sv_b + h * sv_h,
                    sv_t,
                    static_cast<int64_t>(H) * kD,
                    H};

  SoftmaxState st;
  st.init();

  TileRegs<NTHREADS> regs;
  float ksr = 0.f;
  load_tile_i8<BLK, NTHREADS, INT8_PV>(regs, ksr, sh, 0, src, is, T, NT);
  store_tile_i8<BLK, NTHREADS, INT8_PV>(regs, ksr, 0 >= nexact, tbufs[0]);
  __syncthreads();

  for (int n = 0; n < ntiles; ++n) {
    if (n + 1 < ntiles) load_tile_i8<BLK, NTHREADS, INT8_PV>(regs, ksr, sh, n + 1, src, is, T, NT);
    const TileDesc td = tile_desc_i8<BLK>(sh, n, T, NT);
    const TileBuf& tb = tbufs[n & 1];

    if (td.pooled) {
      f32x16 s[2];
      qk_bf16(tb, qreg, col, half, s);
      softmax_update<BLK>(st, s, td, c, half, NT, T);
      pv_bf16(tb, s, col, half, st.acc);
    } else {
      // S^T = Ki . Qi^T (int32), keys 32m + 8(r/4) + 4*half + (r%4).
      i32x16 si[2];
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int r = 0; r < 16; ++r) si[m][r] = 0;
#pragma unroll
      for (int cc = 0; cc < 4; ++cc)
#pragma unroll
        for (int m = 0; m < 2; ++m) {
          const i32x4 a = *reinterpret_cast<const i32x4*>(k_i8(tb) + (32 * m + col) * kKI8Stride +
                                                          cc * 32 + half * 16);
          si[m] = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, qireg[cc], si[m], 0, 0, 0);
        }
      f32x16 s[2];
      float mx = -INFINITY;
      const float* ksl = ks_f(tb);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float4 k4 = *reinterpret_cast<const float4*>(ksl + 32 * m + 8 * i + 4 * half);
          const float kk[4] = {k4.x, k4.y, k4.z, k4.w};
#pragma unroll
          for (int j = 0; j < 4; ++j) {
            const int r = 4 * i + j;
            const int kl = 32 * m + 8 * i + 4 * half + j;
            float sv = static_cast<float>(si[m][r]) * (qsl * kk[j]);
            if (!((td.amask >> kl) & 1ull)) sv = -INFINITY;
            s[m][r] = sv;
            mx = fmaxf(mx, sv);
          }
        }
      const float bmax = fmaxf(mx, __shfl_xor(mx, 32));
      const float m_new = fmaxf(st.m, bmax);
      const float alpha = st.m == m_new ? 1.f : __builtin_amdgcn_exp2f(st.m - m_new);
      if (__any(alpha != 1.f)) {
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r) st.acc[dt][r] *= alpha;
      }
      if constexpr (INT8_PV) {
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
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          i32x16 pv;
#pragma unroll
          for (int r = 0; r < 16; ++r) pv[r] = 0;
#pragma unroll
          for (int kstep = 0; kstep < 2; ++kstep) {
            const i32x4 a = *reinterpret_cast<const i32x4*>(vt_i8(tb) + (32 * dt + col) * kVI8Stride +
                                                            32 * kstep + 16 * half);
            pv = __builtin_amdgcn_mfma_i32_32x32x32_i8(a, pb[kstep], pv, 0, 0, 0);
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
        pv_bf16(tb, s, col, half, st.acc);
      }
      st.m = m_new;
      if (INT8_PV && n == nexact - 1) {
        // Exact phase done: apply the per-channel V scale once.
        const float* vsc = vscale + static_cast<int64_t>(bh) * kD;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            st.acc[dt][r] *= vsc[32 * dt + 8 * (r >> 2) + 4 * half + (r & 3)];
      }
    }

    if (n + 1 < ntiles)
      store_tile_i8<BLK, NTHREADS, INT8_PV>(regs, ksr, n + 1 >= nexact, tbufs[(n + 1) & 1]);
    __syncthreads();
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
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(qi) % 16 == 0 && reinterpret_cast<uintptr_t>(ki) % 16 == 0,
                  SOLATTN_EINVAL, "fwd_int8: qi/ki must be 16-byte aligned");
  if (int8_pv) {
    SOLATTN_REQUIRE(vi && vscale && reinterpret_cast<uintptr_t>(vi) % 16 == 0, SOLATTN_EINVAL,
                    "fwd_int8: int8_pv needs 16-byte aligned vi and vscale");
  } else {
    SOLATTN_REQUIRE(v && reinterpret_cast<uintptr_t>(v) % 16 == 0 && sv_b % 8 == 0 &&
                        sv_t % 8 == 0 && sv_h % 8 == 0,
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
