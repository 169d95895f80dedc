// Building blocks shared by the BF16 and INT8 Sol-Attn forwards on gfx950.
//
// A workgroup serves one query block (BLK rows, BLK/32 waves of 32 rows).
// Its work is a sequence of 64-key tiles: pooled tiles (chunks of 64 pooled
// keys with at least one approximate block) and exact tiles (64 tokens each,
// BLK/64 per exact block, ascending block order). Tiles are staged in LDS,
// double buffered.
#pragma once

#include "common.hpp"

namespace solattn {

constexpr int kKeys = 64;             // keys per tile
constexpr int kD = 128;               // head dim
constexpr int kMaxNT = 2048;          // query/key blocks per head
constexpr int kMaxPool = kMaxNT / 64; // pooled tiles per query block

typedef __attribute__((address_space(3))) void lds_void_t;
typedef __attribute__((address_space(1))) void glb_void_t;

// ----------------------------------------------------------------- tile list
struct TileList {
  uint64_t pmask[kMaxPool];  // approximate-block mask of each pooled tile
  int16_t pchunk[kMaxPool];  // pooled tile -> chunk of 64 pooled keys
  int16_t blist[kMaxNT];     // exact key blocks, ascending
  int npool;
  int nexact;
};

struct KVSource {
  const uint16_t* k;  // token rows (this batch/head)
  int64_t sk;
  const uint16_t* v;
  int64_t sv;
  const uint16_t* kc;  // pooled rows (this batch/head)
  int64_t skc;         // row stride of kc and vc
  const uint16_t* vc;
};

struct TileDesc {
  int pooled;
  int first;       // first token row (exact) or pooled row (pooled)
  int nvalid;      // rows < nvalid are real
  uint64_t amask;  // keys taking part in the softmax
};

// Workgroup -> (batch*head, query block). Workgroups are dealt round-robin to
// the 8 XCDs; remap so each XCD walks a contiguous run of query blocks of the
// same heads, which keeps their K/V blocks in that XCD's L2.
__device__ __forceinline__ void tile_coords(uint32_t w, uint32_t total, int NT, int& bh, int& qb) {
  uint32_t logical = w;
  if ((total & 7u) == 0u) logical = (w & 7u) * (total >> 3) + (w >> 3);
  bh = static_cast<int>(logical / static_cast<uint32_t>(NT));
  qb = static_cast<int>(logical % static_cast<uint32_t>(NT));
}

template <int BLK>
__device__ int build_tile_list(TileList& tl, const int32_t* __restrict__ counts,
                               const int16_t* __restrict__ lists, const uint32_t* __restrict__ mask,
                               int64_t row, int NT, int W, int T) {
  const int cnt = min(max(counts[row], 0), NT);
  for (int e = threadIdx.x; e < cnt; e += blockDim.x) tl.blist[e] = lists[row * NT + e];
  if (threadIdx.x == 0) {
    const uint32_t* mrow = mask + row * W;
    int np = 0;
    for (int c = 0; c * 64 < NT; ++c) {
      uint64_t ex = mrow[2 * c];
      if (2 * c + 1 < W) ex |= static_cast<uint64_t>(mrow[2 * c + 1]) << 32;
      const int nvalid = min(64, NT - 64 * c);
      const uint64_t valid = nvalid >= 64 ? ~0ull : ((1ull << nvalid) - 1ull);
      const uint64_t ap = ~ex & valid;
      if (ap) {
        tl.pmask[np] = ap;
        tl.pchunk[np] = static_cast<int16_t>(c);
        ++np;
      }
    }
    tl.npool = np;
    constexpr int S = BLK / kKeys;
    int ne = cnt * S;
    const int tail = T - (NT - 1) * BLK;
    if (S == 2 && cnt > 0 && lists[row * NT + cnt - 1] == NT - 1 && tail <= kKeys) ne -= 1;
    tl.nexact = ne;
  }
  __syncthreads();
  return tl.npool + tl.nexact;
}

// Tile n: pooled tiles first (n < npool), then exact tiles.
template <int BLK>
__device__ __forceinline__ TileDesc tile_desc(const TileList& tl, int n, int T, int NT) {
  TileDesc td;
  if (n < tl.npool) {
    td.pooled = 1;
    td.first = tl.pchunk[n] * kKeys;
    td.nvalid = min(kKeys, NT - td.first);
    td.amask = tl.pmask[n];
  } else {
    constexpr int S = BLK / kKeys;
    const int e = n - tl.npool;
    const int j = min(max(static_cast<int>(tl.blist[e / S]), 0), NT - 1);
    td.pooled = 0;
    td.first = j * BLK + (e % S) * kKeys;
    td.nvalid = max(0, min(kKeys, T - td.first));
    td.amask = td.nvalid >= kKeys ? ~0ull : ((1ull << td.nvalid) - 1ull);
  }
  return td;
}

// ------------------------------------------------------------- direct tiles
// K and V rows (64 keys x 128 bf16 = 16 chunks of 16 bytes) copied global ->
// LDS without passing through VGPRs. Rows are 256 bytes, one full sweep of the
// 64 four-byte LDS banks, so only the chunk position picks the banks; chunks
// are XOR-swizzled per row:
//   K: physical chunk = chunk ^ (row & 15): a 16-byte operand read serves 16
//      lanes = 16 rows of one chunk per cycle, all in different chunks;
//   V: physical chunk = chunk ^ 4*(row & 3): a ds_read_tr16_b64 serves 32
//      lanes = 4 rows x 4 consecutive chunks per cycle, all distinct.
constexpr int kTileElems = kKeys * kD;  // one K or V tile in LDS (16 KiB)

__device__ __forceinline__ int swz_k(int row, int chunk) { return chunk ^ (row & 15); }
__device__ __forceinline__ int swz_v(int row, int chunk) { return chunk ^ ((row & 3) << 2); }

// Global -> LDS copies (global_load_lds_*): lane i's bytes land at
// lds + size * i, lds wave-uniform (M0). They are issued through inline asm so
// that the compiler does not make later, unrelated LDS reads wait for them;
// every consumer orders them itself: s_waitcnt vmcnt, then a barrier.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p)));
}
// 16 bytes per lane from a per-lane address.
__device__ __forceinline__ void g2l16(const void* g, void* lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds_addr(lds)) : "memory");
}
// 16 bytes per lane from a wave-uniform base plus a 32-bit lane offset.
__device__ __forceinline__ void g2l16_s(const void* base, uint32_t off, void* lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds_addr(lds)) : "memory");
}
// 4 bytes per lane from a per-lane address.
__device__ __forceinline__ void g2l4(const void* g, void* lds) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds_addr(lds)) : "memory");
}

// Issue the copies of tile n into buf. Each instruction moves 64 lanes x 16 B
// into 1 KiB of LDS at (wave base + 16 * lane); lane e of the tile fills
// physical chunk e, so it fetches the logical chunk that lands there. Full
// exact tiles use the per-lane byte offsets precomputed in TileOffsets (tile
// base in SGPRs + 32-bit lane offset); pooled and ragged tiles compute theirs,
// with rows past nvalid re-reading row 0 of the tile (finite data that the
// softmax masks out).
template <int NTHREADS>
struct TileOffsets {
  static constexpr int U = kKeys * 16 / NTHREADS;
  uint32_t k[U], v[U];
  __device__ __forceinline__ void init(int64_t sk, int64_t sv) {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int e = threadIdx.x + NTHREADS * u;
      const int row = e >> 4, pc = e & 15;
      k[u] = static_cast<uint32_t>((row * sk + swz_k(row, pc) * 8) * 2);
      v[u] = static_cast<uint32_t>((row * sv + swz_v(row, pc) * 8) * 2);
    }
  }
};

// Copy the K (kv == 0) or V (kv == 1) rows of the tile `td` into an LDS tile,
// each lane computing its own source rows: rows past nvalid re-read row 0 of
// the tile (finite data that the softmax masks out).
template <int NTHREADS>
__device__ __forceinline__ void issue_generic(uint16_t* dst, int kv, const TileDesc& td,
                                              const KVSource& src) {
  constexpr int U = kKeys * 16 / NTHREADS;
  const int wave_base = threadIdx.x & ~63;
  const uint16_t* b = kv == 0 ? (td.pooled ? src.kc : src.k) : (td.pooled ? src.vc : src.v);
  const int64_t stride = td.pooled ? src.skc : (kv == 0 ? src.sk : src.sv);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = threadIdx.x + NTHREADS * u;
    const int row = e >> 4, pc = e & 15;
    const int srow = td.first + (row < td.nvalid ? row : 0);
    const int chunk = kv == 0 ? swz_k(row, pc) : swz_v(row, pc);
    g2l16(b + static_cast<int64_t>(srow) * stride + chunk * 8, dst + (wave_base + NTHREADS * u) * 8);
  }
}

// As issue_generic, with full exact tiles taking the precomputed lane offsets.
template <int NTHREADS>
__device__ __forceinline__ void issue_desc(uint16_t* dst, int kv, const TileDesc& td,
                                           const KVSource& src, const TileOffsets<NTHREADS>& off) {
  if (!td.pooled && td.nvalid == kKeys) {
    const int wave_base = threadIdx.x & ~63;
    const char* base = kv == 0
        ? reinterpret_cast<const char*>(src.k + static_cast<int64_t>(td.first) * src.sk)
        : reinterpret_cast<const char*>(src.v + static_cast<int64_t>(td.first) * src.sv);
#pragma unroll
    for (int u = 0; u < TileOffsets<NTHREADS>::U; ++u) {
      const int lds_chunk = wave_base + NTHREADS * u;  // first chunk this wave writes
      g2l16(base + (kv == 0 ? off.k[u] : off.v[u]), dst + lds_chunk * 8);
    }
    return;
  }
  issue_generic<NTHREADS>(dst, kv, td, src);
}

// Copy the K (kv == 0) or V (kv == 1) rows of tile n (pooled tiles first) into an LDS tile.
template <int BLK, int NTHREADS>
__device__ __forceinline__ void issue_half(uint16_t* dst, int kv, const TileList& tl, int n,
                                           const KVSource& src, const TileOffsets<NTHREADS>& off,
                                           int T, int NT) {
  issue_desc<NTHREADS>(dst, kv, tile_desc<BLK>(tl, n, T, NT), src, off);
}

__device__ __forceinline__ void wait_tile_copies() { __builtin_amdgcn_s_waitcnt(0); }

// S^T (64 keys x 32 query rows of this wave) = K . Q^T. s[m] covers keys
// 32m + 8(r/4) + 4*half + (r%4) for accumulator element r, query row `col`.
__device__ __forceinline__ void qk_swz(const uint16_t* kt, const bf16x8 (&qreg)[8], int col, int half,
                                       f32x16 (&s)[2]) {
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) s[m][r] = 0.f;
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const int row = 32 * m + col;
      const bf16x8 a =
          *reinterpret_cast<const bf16x8*>(&kt[row * kD + swz_k(row, 2 * cc + half) * 8]);
      s[m] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, qreg[cc], s[m], 0, 0, 0);
    }
  }
}

__device__ __forceinline__ bf16x4 tr16(const uint16_t* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(p));
  return __builtin_bit_cast(bf16x4, r);
}

__device__ __forceinline__ bf16x8 to_bf16x8(const f32x16& s, int off) {
  bf16x8 b;
#pragma unroll
  for (int e = 0; e < 8; ++e) b[e] = static_cast<__bf16>(s[off + e]);
  return b;
}

// O^T += V^T . P^T over the tile's 64 keys, 16 keys per MFMA step. V is
// row-major in LDS; ds_read_tr16_b64 hands lane l the 4 keys
// 16ks + 4*half + k (k = 0..3) of channel 32dt + (l % 32): within each 16-lane
// group, lane s supplies row 16ks + 4*half + s/4, channels 4*(s%4) .. +3.
__device__ __forceinline__ void pv_tr16(const uint16_t* vt, const f32x16 (&p)[2], int lane,
                                        f32x16 (&acc)[4]) {
  const int g = lane >> 4, sl = lane & 15;
  const int half = g >> 1;
  const int sub = sl & 1;                       // 8-byte half of the 16-byte chunk
  const int cpair = 2 * (g & 1) + ((sl & 3) >> 1);
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    const bf16x8 b = to_bf16x8(p[ks >> 1], 8 * (ks & 1));
    const int row0 = 16 * ks + 4 * half + (sl >> 2);
    const int row1 = row0 + 8;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) {
      const int chunk = 4 * dt + cpair;
      const bf16x4 lo = tr16(&vt[row0 * kD + swz_v(row0, chunk) * 8 + sub * 4]);
      const bf16x4 hi = tr16(&vt[row1 * kD + swz_v(row1, chunk) * 8 + sub * 4]);
      const bf16x8 a = __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
      acc[dt] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[dt], 0, 0, 0);
    }
  }
}

// ------------------------------------------------------------ online softmax
constexpr float kMaxSlack = 8.f;

struct SoftmaxState {
  float m;          // running max, in the exp2 domain (score * c)
  float l;          // partial row sum over this lane's keys
  f32x16 acc[4];    // O^T: channel 32dt + 8(r/4) + 4*half + (r%4), query row `col`
  __device__ __forceinline__ void init() {
    m = -INFINITY;
    l = 0.f;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[dt][r] = 0.f;
  }
};

// Online softmax over one tile: p = exp2(s*c - m_new) replaces s in place.
// Pooled keys carry weight len_j in the row sum (/root/reference/_tri_fwd.py:302-307).
template <int BLK>
__device__ __forceinline__ void softmax_update(SoftmaxState& st, f32x16 (&s)[2], const TileDesc& td,
                                               float c, int half, int NT, int T) {
  if (td.amask != ~0ull) {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kl = 32 * m + 8 * (r >> 2) + 4 * half + (r & 3);
        if (!((td.amask >> kl) & 1ull)) s[m][r] = -INFINITY;
      }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[m][r]);
  mx = fmaxf(mx, __shfl_xor(mx, 32));
  // The running max moves only when the tile's max exceeds it by more than
  // kMaxSlack (log2 units): p may then reach 2^kMaxSlack, harmless in bf16 P
  // and fp32 sums, and the O rescale becomes rare.
  const float m_tile = mx * c;
  const float m_new = m_tile > st.m + kMaxSlack ? m_tile : st.m;
  const float alpha = st.m == m_new ? 1.f : __builtin_amdgcn_exp2f(st.m - m_new);
  const float neg = -m_new;
  float psum = 0.f;
  if (td.pooled) {
    const int tail = T - (NT - 1) * BLK;
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kl = 32 * m + 8 * (r >> 2) + 4 * half + (r & 3);
        const float p = __builtin_amdgcn_exp2f(fmaf(s[m][r], c, neg));
        s[m][r] = p;
        const float w = (td.first + kl == NT - 1) ? static_cast<float>(tail) : static_cast<float>(BLK);
        psum = fmaf(p, w, psum);
      }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float p = __builtin_amdgcn_exp2f(fmaf(s[m][r], c, neg));
        s[m][r] = p;
        psum += p;
      }
  }
  st.l = fmaf(st.l, alpha, psum);
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[dt][r] *= alpha;
  }
  st.m = m_new;
}

// o[qrow, :] = acc / l (bf16), rows past T skipped.
__device__ __forceinline__ void store_output(const SoftmaxState& st, uint16_t* __restrict__ obase,
                                             int64_t so_t, int qrow, int T, int half) {
  const float l = st.l + __shfl_xor(st.l, 32);
  const float inv = 1.f / l;
  if (qrow >= T) return;
  uint16_t* orow = obase + static_cast<int64_t>(qrow) * so_t;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      uint2 w;
      w.x = pack_bf16x2(st.acc[dt][4 * i] * inv, st.acc[dt][4 * i + 1] * inv);
      w.y = pack_bf16x2(st.acc[dt][4 * i + 2] * inv, st.acc[dt][4 * i + 3] * inv);
      *reinterpret_cast<uint2*>(orow + 32 * dt + 8 * i + 4 * half) = w;
    }
}

// ------------------------------------------------------------ argument checks
inline int check_fwd_common(const void* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                            const void* kc, const void* vc, int64_t npad, const int32_t* counts,
                            const int16_t* lists, const uint32_t* mask, int64_t B, int64_t T,
                            int64_t H, int64_t D, int64_t block, const void* o, int64_t so_b,
                            int64_t so_t, int64_t so_h, const char* what) {
  SOLATTN_REQUIRE(D == kD, SOLATTN_EUNSUPPORTED, "%s: head_dim %lld != 128", what, (long long)D);
  SOLATTN_REQUIRE(block == 64 || block == 128, SOLATTN_EUNSUPPORTED, "%s: block %lld not in {64, 128}",
                  what, (long long)block);
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0, SOLATTN_EINVAL, "%s: bad sizes", what);
  const int64_t NT = cdiv(T, block);
  SOLATTN_REQUIRE(NT <= kMaxNT, SOLATTN_EUNSUPPORTED, "%s: %lld blocks exceed %d", what,
                  (long long)NT, kMaxNT);
  SOLATTN_REQUIRE(B * H * NT < (1ll << 31), SOLATTN_EUNSUPPORTED, "%s: grid too large", what);
  SOLATTN_REQUIRE(npad >= cdiv(NT, 64) * 64, SOLATTN_EINVAL,
                  "%s: npad %lld must cover whole 64-block chunks", what, (long long)npad);
  SOLATTN_REQUIRE(q && kc && vc && counts && lists && mask && o, SOLATTN_EINVAL, "%s: null pointer",
                  what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && sq_b % 8 == 0 && sq_t % 8 == 0 &&
                      sq_h % 8 == 0,
                  SOLATTN_EINVAL, "%s: q must be 16-byte aligned with strides multiple of 8", what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(kc) % 16 == 0 && reinterpret_cast<uintptr_t>(vc) % 16 == 0,
                  SOLATTN_EINVAL, "%s: kc/vc must be 16-byte aligned", what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(o) % 8 == 0 && so_b % 4 == 0 && so_t % 4 == 0 &&
                      so_h % 4 == 0,
                  SOLATTN_EINVAL, "%s: o must be 8-byte aligned with strides multiple of 4", what);
  return 0;
}

inline int check_fwd_args(const void* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const void* k,
                          int64_t sk_b, int64_t sk_t, int64_t sk_h, const void* v, int64_t sv_b,
                          int64_t sv_t, int64_t sv_h, const void* kc, const void* vc, int64_t npad,
                          const int32_t* counts, const int16_t* lists, const uint32_t* mask,
                          int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, const void* o,
                          int64_t so_b, int64_t so_t, int64_t so_h, const char* what) {
  if (int rc = check_fwd_common(q, sq_b, sq_t, sq_h, kc, vc, npad, counts, lists, mask, B, T, H, D,
                                block, o, so_b, so_t, so_h, what))
    return rc;
  SOLATTN_REQUIRE(k && v, SOLATTN_EINVAL, "%s: null k/v", what);
  // Lane offsets within a 64-row tile are kept in 32 bits.
  SOLATTN_REQUIRE(sk_t >= 0 && sv_t >= 0 && sk_t < (1ll << 24) && sv_t < (1ll << 24),
                  SOLATTN_EUNSUPPORTED, "%s: token strides beyond 2^24 elements", what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(k) % 16 == 0 && sk_b % 8 == 0 && sk_t % 8 == 0 &&
                      sk_h % 8 == 0 && reinterpret_cast<uintptr_t>(v) % 16 == 0 && sv_b % 8 == 0 &&
                      sv_t % 8 == 0 && sv_h % 8 == 0,
                  SOLATTN_EINVAL, "%s: k/v must be 16-byte aligned with strides multiple of 8", what);
  return 0;
}

}  // namespace solattn
