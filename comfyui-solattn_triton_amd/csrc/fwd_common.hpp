// Building blocks shared by the BF16 and INT8 Sol-Attn forwards on gfx950.
//
// A workgroup serves one query block (BLK rows, BLK/32 waves of 32 rows, two
// workgroups per CU). Its work is a sequence of 64-key tiles: pooled tiles
// (chunks of 64 pooled keys with at least one approximate block) and exact
// tiles (64 tokens each, BLK/64 per exact block, ascending block order).
// Tiles are copied global -> LDS (double buffered) and consumed by MFMA:
//   S^T = K . Q^T (v_mfma_f32_32x32x16_bf16): lane l holds query row l%32 and
//     keys 32m + 8(r/4) + 4(l/32) + r%4 in element r of tile m, so row max and
//     sum need one exchange between lanes 32 apart;
//   O^T += V^T . P^T: the S accumulator converts in place into the B operand;
//     V stays row-major in LDS and ds_read_b64_tr_b16 delivers V^T with the
//     matching key order.
#pragma once

#include "common.hpp"

namespace solattn {

constexpr int kKeys = 64;             // keys per tile
constexpr int kD = 128;               // head dim
constexpr int kMaxNT = 16384;         // query/key blocks per head
constexpr int kMaxPool = kMaxNT / 64; // pooled tiles per query block
constexpr float kMaxSlack = 8.f;      // lazy running max (log2 units)

// ----------------------------------------------------------------- tile list
struct TileList {
  uint64_t pmask[kMaxPool];  // approximate-block mask of each pooled tile
  int16_t pchunk[kMaxPool];  // pooled tile -> chunk of 64 pooled keys
  int npool;   // pooled tiles
  int nexact;  // exact 64-key tiles
  int nblk;    // exact key blocks (the first nblk entries of blist_lds())
  int last;    // highest exact key block, -1 if none
};

// The exact key blocks of the workgroup's query block, ascending, live in the
// launch's dynamic LDS (blist_lds_bytes(NT) bytes), so a short sequence does
// not pay LDS for the longest one.
__device__ __forceinline__ int16_t* blist_lds() {
  extern __shared__ __align__(16) int16_t solattn_blist[];
  return solattn_blist;
}
inline size_t blist_lds_bytes(int64_t NT) { return static_cast<size_t>(cdiv(NT * 2, 16) * 16); }

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
// the 8 XCDs; they are remapped so that each XCD walks a contiguous run of
// query blocks of the same heads, which keeps their K/V blocks in that XCD's
// L2. Within each window of WIN consecutive dispatches on an XCD (the query
// blocks that run there together) the query blocks are taken longest first,
// by exact-block count: the window's counts are ranked in LDS and this
// workgroup takes the query block whose rank is its place in the window. Same
// L2 footprint, shorter tail per window (4-9% faster forwards at cfg 2). A
// window spans kLptTokens query tokens: 64 dispatches at block 128, 128 at
// block 64 (a 128-dispatch window is 3-4% faster than 64 at block 64, and
// 256 is slower at both sizes).
constexpr int kLptTokens = 8192;
template <int WIN>
__device__ __forceinline__ void tile_coords_lpt(const int32_t* __restrict__ counts, int NT, int& bh,
                                                int& qb) {
  static_assert(WIN > 0 && (WIN & (WIN - 1)) == 0, "window offsets are taken with masks");
  __shared__ int s_cnt[WIN];
  __shared__ int s_pick;
  const uint32_t w = blockIdx.x, total = gridDim.x;
  uint32_t base, r, nwin;
  if ((total & 7u) == 0u) {
    const uint32_t per = total >> 3, li = w >> 3;
    base = (w & 7u) * per + (li & ~(WIN - 1u));
    r = li & (WIN - 1u);
    nwin = min(static_cast<uint32_t>(WIN), per - (li & ~(WIN - 1u)));
  } else {
    base = w & ~(WIN - 1u);
    r = w & (WIN - 1u);
    nwin = min(static_cast<uint32_t>(WIN), total - base);
  }
  // Strided over the workgroup so that every window slot is filled and ranked
  // whatever the thread count; exactly one slot has rank r, so s_pick is set.
  for (int t = threadIdx.x; t < WIN; t += blockDim.x)
    s_cnt[t] = t < static_cast<int>(nwin) ? counts[base + t] : -1;
  __syncthreads();
  for (int t = threadIdx.x; t < static_cast<int>(nwin); t += blockDim.x) {
    const int mine = s_cnt[t];
    int rank = 0;
    for (int u = 0; u < static_cast<int>(nwin); ++u) {
      const int cu = s_cnt[u];
      rank += (cu > mine) || (cu == mine && u < t);
    }
    if (rank == static_cast<int>(r)) s_pick = t;
  }
  __syncthreads();
  const uint32_t logical = base + static_cast<uint32_t>(s_pick);
  bh = static_cast<int>(logical / static_cast<uint32_t>(NT));
  qb = static_cast<int>(logical % static_cast<uint32_t>(NT));
}

// The workgroup's tiles, from its row of the routing bitmask (bit j of word
// j/32 = key block j is exact). Needs at least two waves: wave 0 collects the
// pooled chunks, wave 1 the exact blocks, in parallel. Every entry comes from
// a set bit below NT, so any mask contents give in-range tiles.
template <int BLK>
__device__ int build_tile_list(TileList& tl, const uint32_t* __restrict__ mask, int64_t row,
                               int NT, int W, int T) {
  const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t* mrow = mask + row * W;
  if (wave == 0) {
    // Pooled chunks (64 key blocks each): one chunk per lane, 64 chunks a
    // pass, so the mask words are loaded together; a ballot prefix keeps the
    // chunks in ascending order.
    int np = 0;
    for (int c0 = 0; c0 * 64 < NT; c0 += 64) {
      const int c = c0 + lane;
      uint64_t ap = 0;
      if (c * 64 < NT) {
        uint64_t ex = mrow[2 * c];
        if (2 * c + 1 < W) ex |= static_cast<uint64_t>(mrow[2 * c + 1]) << 32;
        const int nvalid = min(64, NT - 64 * c);
        const uint64_t valid = nvalid >= 64 ? ~0ull : ((1ull << nvalid) - 1ull);
        ap = ~ex & valid;
      }
      const uint64_t has = __ballot(ap != 0ull);
      if (ap) {
        const int pos = np + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(has >> 32),
                                                       __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(has), 0));
        tl.pmask[pos] = ap;
        tl.pchunk[pos] = static_cast<int16_t>(c);
      }
      np += __popcll(has);
    }
    if (lane == 0) tl.npool = np;
  } else if (wave == 1) {
    // Exact blocks, ascending: one lane per block, 64 blocks per ballot. The
    // words of 2048 blocks come in one load per lane and are passed around
    // with shuffles.
    int16_t* blist = blist_lds();
    int ne = 0, last = -1;
    for (int w0 = 0; w0 < W; w0 += 64) {
      const uint32_t word = w0 + lane < W ? mrow[w0 + lane] : 0u;
      const int nw = min(64, W - w0);
      for (int p = 0; 2 * p < nw; ++p) {
        const uint32_t mine = __shfl(word, 2 * p + (lane >> 5));
        const int j = (w0 + 2 * p) * 32 + lane;
        const bool ex = j < NT && ((mine >> (lane & 31)) & 1u);
        const uint64_t bal = __ballot(ex);
        if (ex)
          blist[ne + __builtin_amdgcn_mbcnt_hi(static_cast<uint32_t>(bal >> 32),
                                               __builtin_amdgcn_mbcnt_lo(static_cast<uint32_t>(bal), 0))] =
              static_cast<int16_t>(j);
        ne += __popcll(bal);
        if (bal) last = (w0 + 2 * p) * 32 + 63 - __clzll(bal);
      }
    }
    if (lane == 0) {
      constexpr int S = BLK / kKeys;
      const int tail = T - (NT - 1) * BLK;
      tl.nblk = ne;
      tl.last = last;
      // at block 128 a last block of at most 64 tokens is one (ragged) tile
      tl.nexact = ne * S - ((S == 2 && last == NT - 1 && tail <= kKeys) ? 1 : 0);
    }
  }
  __syncthreads();  // the lists and counts are in LDS
  return tl.npool + tl.nexact;
}

// The last exact tile is ragged when block NT-1 is exact and T is not a
// multiple of 64 (exact blocks are listed in ascending order).
__device__ __forceinline__ int ragged_tiles(const TileList& tl, int NT, int T) {
  return (tl.nexact > 0 && tl.last == NT - 1 && (T % kKeys) != 0) ? 1 : 0;
}

// Pooled tile p.
__device__ __forceinline__ TileDesc pooled_desc(const TileList& tl, int p, int NT) {
  TileDesc td;
  td.pooled = 1;
  td.first = tl.pchunk[p] * kKeys;
  td.nvalid = min(kKeys, NT - td.first);
  td.amask = tl.pmask[p];
  return td;
}

// Exact tile e (list order).
template <int BLK>
__device__ __forceinline__ TileDesc exact_desc(const TileList& tl, int e, int T, int NT) {
  constexpr int S = BLK / kKeys;
  const int j = min(max(static_cast<int>(blist_lds()[e / S]), 0), NT - 1);
  TileDesc td;
  td.pooled = 0;
  td.first = j * BLK + (e % S) * kKeys;
  td.nvalid = max(0, min(kKeys, T - td.first));
  td.amask = td.nvalid >= kKeys ? ~0ull : ((1ull << td.nvalid) - 1ull);
  return td;
}

// First token row of full exact tile e (list order), wave-uniform.
template <int BLK>
__device__ __forceinline__ int exact_first(const TileList& tl, int e) {
  constexpr int S = BLK / kKeys;
  const int j = blist_lds()[e / S];
  return __builtin_amdgcn_readfirstlane(j * BLK + (e % S) * kKeys);
}

// ------------------------------------------------------------- LDS copies
// K and V rows (64 keys x 128 bf16 = 16 chunks of 16 bytes) land in LDS rows
// of 256 bytes, one full sweep of the 64 four-byte banks, so only the chunk
// position picks the banks; chunks are XOR-swizzled per row:
//   K: physical chunk = chunk ^ (row & 15): a 16-byte operand read serves 16
//      lanes = 16 rows of one chunk per cycle, all in different chunks;
//   V: physical chunk = chunk ^ 4*(row & 3): a ds_read_b64_tr_b16 serves 32
//      lanes = 4 rows x 4 consecutive chunks per cycle, all distinct.
constexpr int kTileElems = kKeys * kD;  // one K or V tile in LDS (16 KiB)
constexpr uint32_t kTileBytes = kTileElems * 2;

__device__ __forceinline__ int swz_k(int row, int chunk) { return chunk ^ (row & 15); }
__device__ __forceinline__ int swz_v(int row, int chunk) { return chunk ^ ((row & 3) << 2); }

// Global -> LDS copies (global_load_lds_*): lane i's bytes land at
// lds + size * i, with lds a wave-uniform LDS byte address (M0). They are
// issued through inline asm so that the compiler does not make later,
// unrelated LDS reads wait for them; every consumer orders them itself:
// s_waitcnt vmcnt, then a barrier. Callers convert the LDS pointer once
// (lds_addr) and add scalar offsets, so the addresses stay in SGPRs.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return __builtin_amdgcn_readfirstlane(
      static_cast<uint32_t>(reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) char*)p)));
}
// This wave's index in the workgroup, as a scalar.
__device__ __forceinline__ int wave_id() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x) >> 6);
}
// 16 bytes per lane from a per-lane address.
__device__ __forceinline__ void g2l16(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
// 16 bytes per lane from a wave-uniform base plus a 32-bit lane offset.
__device__ __forceinline__ void g2l16_s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("global_load_lds_dwordx4 %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}
// 4 bytes per lane from a per-lane address.
__device__ __forceinline__ void g2l4(const void* g, uint32_t lds) {
  asm volatile("global_load_lds_dword %0, off" ::"v"(g), "{m0}"(lds) : "memory");
}
// 4 bytes per lane from a wave-uniform base plus a 32-bit lane offset.
__device__ __forceinline__ void g2l4_s(const void* base, uint32_t off, uint32_t lds) {
  asm volatile("global_load_lds_dword %0, %1" ::"v"(off), "s"(base), "{m0}"(lds) : "memory");
}

__device__ __forceinline__ void wait_tile_copies() { __builtin_amdgcn_s_waitcnt(0); }

// s_waitcnt vmcnt(N): all but the N newest copies have landed (vmcnt is bits
// [3:0] and [15:14]; expcnt and lgkmcnt stay at their maxima).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt is 6 bits");
  __builtin_amdgcn_s_waitcnt((N & 15) | ((N >> 4) << 14) | 0x0f70);
}

// Copy the K (kv == 0) or V (kv == 1) rows of the bf16 tile `td` into an LDS
// tile, each lane computing its own source rows: rows past nvalid re-read row
// 0 of the tile (finite data that the softmax masks out). U copies per lane.
// dst is the tile's LDS byte address.
template <int NTHREADS>
__device__ __forceinline__ void issue_generic(uint32_t dst, int kv, const TileDesc& td,
                                              const KVSource& src) {
  constexpr int U = kKeys * 16 / NTHREADS;
  const uint32_t l0 = dst + wave_id() * 64 * 16;
  const uint16_t* b = kv == 0 ? (td.pooled ? src.kc : src.k) : (td.pooled ? src.vc : src.v);
  const int64_t stride = td.pooled ? src.skc : (kv == 0 ? src.sk : src.sv);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int e = threadIdx.x + NTHREADS * u;
    const int row = e >> 4, pc = e & 15;
    const int srow = td.first + (row < td.nvalid ? row : 0);
    const int chunk = kv == 0 ? swz_k(row, pc) : swz_v(row, pc);
    g2l16(b + static_cast<int64_t>(srow) * stride + chunk * 8, l0 + NTHREADS * u * 16);
  }
}

// Per-lane byte offsets of the 16-byte chunks this lane copies into a full
// bf16 K or V tile. Copy u covers rows (NTHREADS/16)u ..; lanes repeat their
// swizzle every P copies (P = 256 / NTHREADS), so the offset of copy u is
// off[u % P] + (u / P) * 16 * row stride, the second term wave-uniform.
template <int NTHREADS>
struct CopyOffsets {
  static constexpr int U = kKeys * 16 / NTHREADS;  // copies per lane per K or V tile
  static constexpr int P = 256 / NTHREADS;
  uint32_t k[P], v[P];
  __device__ __forceinline__ void init(int64_t sk, int64_t sv) {
#pragma unroll
    for (int u = 0; u < P; ++u) {
      const int e = threadIdx.x + NTHREADS * u;
      const int row = e >> 4, pc = e & 15;
      k[u] = static_cast<uint32_t>((row * sk + swz_k(row, pc) * 8) * 2);
      v[u] = static_cast<uint32_t>((row * sv + swz_v(row, pc) * 8) * 2);
    }
  }
};

// Copies of a full bf16 tile whose first row is at `base` (row stride
// `stride` elements) into the LDS tile at byte address dst.
template <int NTHREADS>
__device__ __forceinline__ void issue_full(uint32_t dst, const uint16_t* base, int64_t stride,
                                           const uint32_t (&off)[CopyOffsets<NTHREADS>::P]) {
  using CO = CopyOffsets<NTHREADS>;
  const uint32_t l0 = dst + wave_id() * 64 * 16;
  const char* b = reinterpret_cast<const char*>(base);
#pragma unroll
  for (int u = 0; u < CO::U; ++u) {
    const char* row_base = b + static_cast<int64_t>(u / CO::P) * 16 * stride * 2;
    g2l16_s(row_base, off[u % CO::P], l0 + NTHREADS * u * 16);
  }
}

// ------------------------------------------------------------ bf16 MFMA tiles
__device__ __forceinline__ f32x16 mfma_bf16(const bf16x8& a, const bf16x8& b, const f32x16& c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ bf16x4 tr16(const uint16_t* p) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const v4i16 r = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      (__attribute__((address_space(3))) v4i16*)(p));
  return __builtin_bit_cast(bf16x4, r);
}

// K operand of S^T = K . Q^T: key 32m + col, dims 16cc + 8half .. +7.
__device__ __forceinline__ bf16x8 k_op(const uint16_t* kt, int m, int cc, int col, int half) {
  const int row = 32 * m + col;
  return *reinterpret_cast<const bf16x8*>(&kt[row * kD + swz_k(row, 2 * cc + half) * 8]);
}

// V^T operand of O^T += V^T . P^T for key step ks (16 keys) and channel tile
// dt: lane l gets channel 32dt + l%32 of keys 16ks + 8(e/4) + 4(l/32) + e%4,
// the key order of S accumulator elements 8(ks%2) .. +7 of tile ks/2. Within
// a 16-lane group, lane s of the ds_read_b64_tr_b16 supplies row
// 16ks + 4(l/32) + s/4 (+8 for the second read), channels 4(s%4) .. +3.
__device__ __forceinline__ bf16x8 v_op(const uint16_t* vt, int ks, int dt, int lane) {
  const int g = lane >> 4, sl = lane & 15;
  const int half = g >> 1;
  const int sub = sl & 1;
  const int chunk = 4 * dt + 2 * (g & 1) + ((sl & 3) >> 1);
  const int row0 = 16 * ks + 4 * half + (sl >> 2);
  const int row1 = row0 + 8;
  const bf16x4 lo = tr16(&vt[row0 * kD + swz_v(row0, chunk) * 8 + sub * 4]);
  const bf16x4 hi = tr16(&vt[row1 * kD + swz_v(row1, chunk) * 8 + sub * 4]);
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}

// Operand addressing by XOR. In a 256-byte-aligned K tile the operand (m, cc)
// of a lane sits at (k_lane ^ (cc << 5)) + m * 8192, because the swizzle
// c ^ (row & 15) only flips chunk bits that cc's chunk index 2cc + half
// shares with bits 5-7 of the address. In a V tile the transposed operand
// (ks, dt) rows row0 / row0 + 8 sit at (v_lane ^ (dt << 6)) + ks * 4096 and
// 2048 further (swizzle c ^ ((row & 3) << 2) flips address bits 6-7). One
// lane address per tile replaces one per (cc) or (dt).
__device__ __forceinline__ uint32_t k_lane(uint32_t tile, int col, int half) {
  return tile + col * 256 + 16 * (half ^ (col & 15));
}
__device__ __forceinline__ uint32_t v_lane(uint32_t tile, int lane) {
  const int g = lane >> 4, sl = lane & 15;
  const int row0 = 4 * (g >> 1) + (sl >> 2);
  const int cp = 2 * (g & 1) + ((sl & 3) >> 1);
  return tile + row0 * 256 + 64 * (row0 & 3) + 16 * cp + 8 * (sl & 1);
}
__device__ __forceinline__ bf16x8 k_op_x(uint32_t kl, int m, int cc) {
  const uint32_t a = (kl ^ static_cast<uint32_t>(cc << 5)) + m * 8192;
  return *reinterpret_cast<const __attribute__((address_space(3))) bf16x8*>(static_cast<uintptr_t>(a));
}
__device__ __forceinline__ bf16x8 v_op_x(uint32_t vl, int ks, int dt) {
  typedef short v4i16 __attribute__((ext_vector_type(4)));
  const uint32_t a = (vl ^ static_cast<uint32_t>(dt << 6)) + ks * 4096;
  const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) v4i16*>(static_cast<uintptr_t>(a)));
  const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
      reinterpret_cast<__attribute__((address_space(3))) v4i16*>(static_cast<uintptr_t>(a + 2048)));
  return __builtin_bit_cast(bf16x8, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

__device__ __forceinline__ void qk_tile(const uint16_t* kt, const bf16x8 (&q)[8], int col, int half,
                                        f32x16 (&s)[2]) {
  const f32x16 zero = {};
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    const bf16x8 a0 = k_op(kt, 0, cc, col, half);
    const bf16x8 a1 = k_op(kt, 1, cc, col, half);
    s[0] = mfma_bf16(a0, q[cc], cc == 0 ? zero : s[0]);
    s[1] = mfma_bf16(a1, q[cc], cc == 0 ? zero : s[1]);
  }
}

// O^T += V^T . P^T over the tile's 16 (key step, channel tile) operands, each
// read three operands ahead of its MFMA.
// The same from the lane address kl = k_lane(tile, col, half) of a
// 256-byte-aligned K tile: no per-chunk addresses to keep live.
__device__ __forceinline__ void qk_tile(uint32_t kl, const bf16x8 (&q)[8], f32x16 (&s)[2]) {
  const f32x16 zero = {};
#pragma unroll
  for (int cc = 0; cc < 8; ++cc) {
    const bf16x8 a0 = k_op_x(kl, 0, cc);
    const bf16x8 a1 = k_op_x(kl, 1, cc);
    s[0] = mfma_bf16(a0, q[cc], cc == 0 ? zero : s[0]);
    s[1] = mfma_bf16(a1, q[cc], cc == 0 ? zero : s[1]);
  }
}

// O^T += V^T . P^T over one tile; vop(ks, dt) gives the V^T operand.
template <typename VOp>
__device__ __forceinline__ void pv_tile_with(VOp&& vop, const bf16x8 (&pb)[4], f32x16 (&o)[4]) {
  constexpr int L = 3;
  bf16x8 va[16];
#pragma unroll
  for (int i = 0; i < L; ++i) va[i] = vop(i >> 2, i & 3);
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    if (i + L < 16) va[i + L] = vop((i + L) >> 2, (i + L) & 3);
    o[i & 3] = mfma_bf16(va[i], pb[i >> 2], o[i & 3]);
  }
}
__device__ __forceinline__ void pv_tile(const uint16_t* vt, const bf16x8 (&pb)[4], int lane,
                                        f32x16 (&o)[4]) {
  pv_tile_with([&](int ks, int dt) { return v_op(vt, ks, dt, lane); }, pb, o);
}
// From the lane address vl = v_lane(tile, lane) of a 256-byte-aligned V tile.
__device__ __forceinline__ void pv_tile(uint32_t vl, const bf16x8 (&pb)[4], int /*lane*/,
                                        f32x16 (&o)[4]) {
  pv_tile_with([&](int ks, int dt) { return v_op_x(vl, ks, dt); }, pb, o);
}

// ------------------------------------------- hand-ordered MFMA / softmax stream
// The pipelined step issues its MFMAs and its softmax as inline asm so that
// the instruction order is the one written: one MFMA, one pair of exps, the
// next MFMA. (Left to the compiler, the MFMAs go out four at a time with ~30
// VALU instructions behind them, and the MFMA pipe idles during the softmax.)
// The compiler does not know that these asm statements are MFMAs, so the
// hazards it would cover with wait states are covered here:
//   VALU write -> MFMA read of that VGPR: 2 wait states, the s_nop 2 in front
//     of the first P.V MFMA of a step (P and the rescaled O are written by
//     VALU code before it);
//   MFMA write -> VALU read of the result: at most NumPasses + 4 = 12 wait
//     states for these 8-pass MFMAs; scores reach the softmax only through
//     mfma_fence (16 wait states) or the in-out operands of the last MFMA
//     of a step, which follows the last score MFMA by a pair of exps and
//     another MFMA.
// Every statement is volatile, so they keep their program order.
__device__ __forceinline__ void mfma_v0(f32x16& d, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, 0" : "=&v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_v(f32x16& d, const bf16x8& a, const bf16x8& b) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
__device__ __forceinline__ void mfma_v_first(f32x16& d, const bf16x8& a, const bf16x8& b) {
  asm volatile("s_nop 2\n\tv_mfma_f32_32x32x16_bf16 %0, %1, %2, %0" : "+v"(d) : "v"(a), "v"(b));
}
// An MFMA that also passes s through: readers of s come after it.
__device__ __forceinline__ void mfma_v_tie(f32x16& d, const bf16x8& a, const bf16x8& b,
                                           f32x16 (&s)[2]) {
  asm volatile("v_mfma_f32_32x32x16_bf16 %0, %3, %4, %0\n\ts_nop 3"
               : "+v"(d), "+v"(s[0]), "+v"(s[1])
               : "v"(a), "v"(b));
}
// 16 wait states after the MFMAs that wrote x; readers of x come after it.
template <int N>
__device__ __forceinline__ void mfma_fence(f32x16 (&x)[N]) {
  static_assert(N == 2 || N == 4, "fence sizes");
  if constexpr (N == 2)
    asm volatile("s_nop 7\n\ts_nop 7" : "+v"(x[0]), "+v"(x[1]));
  else
    asm volatile("s_nop 7\n\ts_nop 7" : "+v"(x[0]), "+v"(x[1]), "+v"(x[2]), "+v"(x[3]));
}
// p = exp2(s*c + neg) for two scores, packed to bf16 (round to nearest even)
// and added to the row sum as packed, one v_dot2_f32_bf16 against (1, 1): the
// denominator is the sum of the P that the P.V MFMA multiplies (the
// reference sums the fp32 p, /root/reference/_tri_fwd.py:330; the difference
// is the bf16 rounding of P, already in the numerator). The s_nop covers the
// one wait state a transcendental result needs before a VALU reads it.
__device__ __forceinline__ uint32_t exp_pair(float s0, float s1, float c, float neg, float& sum) {
  uint32_t p;
  float t0, t1;
  asm volatile(
      "v_fma_f32 %2, %4, %6, %7\n\t"
      "v_fma_f32 %3, %5, %6, %7\n\t"
      "v_exp_f32 %2, %2\n\t"
      "v_exp_f32 %3, %3\n\t"
      "s_nop 0\n\t"
      "v_cvt_pk_bf16_f32 %0, %2, %3\n\t"
      "v_dot2_f32_bf16 %1, %0, %8, %1"
      : "=&v"(p), "+v"(sum), "=&v"(t0), "=&v"(t1)
      : "v"(s0), "v"(s1), "v"(c), "v"(neg), "s"(0x3F803F80u));
  return p;
}
// ------------------------------------------------------------ online softmax
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

// x combined with the value of the lane 32 apart (one v_permlane32_swap).
__device__ __forceinline__ float xhalf_max(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float xhalf_sum(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Running-max update: the max moves only when the tile max exceeds it by more
// than kMaxSlack (log2 units), so p may reach 2^kMaxSlack (harmless in bf16 P
// and fp32 sums) and the O rescale is rare.
__device__ __forceinline__ float new_max(float m_old, float m_tile, float& alpha) {
  const float m_new = m_tile > m_old + kMaxSlack ? m_tile : m_old;
  alpha = m_old == m_new ? 1.f : __builtin_amdgcn_exp2f(m_old - m_new);
  return m_new;
}

// p = exp2(s*c + neg) for elements [R0, R0 + 8) of s, packed to bf16 into pk;
// the row sum accumulates the packed values (v_dot2 with ones), as exp_pair
// (the plain path and the pipelined steps' rare recompute).
template <int R0>
__device__ __forceinline__ float exp8(const f32x16& s, float c, float neg, bf16x8& pk, float sum) {
  const bf16x2 ones = {static_cast<__bf16>(1.f), static_cast<__bf16>(1.f)};
#pragma unroll
  for (int e = 0; e < 8; e += 2) {
    bf16x2 two;
    two[0] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(s[R0 + e], c, neg)));
    two[1] = static_cast<__bf16>(__builtin_amdgcn_exp2f(fmaf(s[R0 + e + 1], c, neg)));
    pk[e] = two[0];
    pk[e + 1] = two[1];
    sum = __builtin_amdgcn_fdot2_f32_bf16(two, ones, sum, false);
  }
  return sum;
}

__device__ __forceinline__ void rescale(SoftmaxState& st, float alpha) {
  if (__any(alpha != 1.f)) {
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 16; ++r) st.acc[dt][r] *= alpha;
  }
}

// Softmax and P.V of one bf16 tile whose scores are in s (the plain path:
// pooled, ragged and last tiles). Masked keys get -inf; pooled keys weigh
// len_j in the row sum (/root/reference/_tri_fwd.py:302-307); P is rounded to
// bf16 for the MFMA and, for exact tiles, summed as rounded (as on the
// pipelined path).
// vt: the V tile, as a pointer or as the lane address v_lane(tile, lane) of a
// 256-byte-aligned tile (see pv_tile).
template <int BLK, typename VTile>
__device__ __forceinline__ void finish_tile(SoftmaxState& st, f32x16 (&s)[2], VTile vt,
                                            const TileDesc& td, float c, int lane, int NT, int T) {
  const int half = lane >> 5;
  if (td.amask != ~0ull) {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      const uint32_t bits = static_cast<uint32_t>(td.amask >> (32 * m + 4 * half));
#pragma unroll
      for (int r = 0; r < 16; ++r)
        s[m][r] = ((bits >> (8 * (r >> 2) + (r & 3))) & 1u) ? s[m][r] : -INFINITY;
    }
  }
  float mx = -INFINITY;
#pragma unroll
  for (int m = 0; m < 2; ++m)
#pragma unroll
    for (int r = 0; r < 16; ++r) mx = fmaxf(mx, s[m][r]);
  float alpha;
  st.m = new_max(st.m, xhalf_max(mx) * c, alpha);
  const float neg = -st.m;
  bf16x8 pb[4];
  float psum = 0.f;
  if (td.pooled) {
    const int kl_last = NT - 1 - td.first;
    const float tail = static_cast<float>(T - (NT - 1) * BLK);
#pragma unroll
    for (int m = 0; m < 2; ++m)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int kl = 32 * m + 8 * (r >> 2) + 4 * half + (r & 3);
        const float p = __builtin_amdgcn_exp2f(fmaf(s[m][r], c, neg));
        pb[2 * m + (r >> 3)][r & 7] = static_cast<__bf16>(p);
        psum = fmaf(p, kl == kl_last ? tail : static_cast<float>(BLK), psum);
      }
  } else {
#pragma unroll
    for (int m = 0; m < 2; ++m) {
      psum = exp8<0>(s[m], c, neg, pb[2 * m], psum);
      psum = exp8<8>(s[m], c, neg, pb[2 * m + 1], psum);
    }
  }
  st.l = fmaf(st.l, alpha, psum);
  rescale(st, alpha);
  pv_tile(vt, pb, lane, st.acc);
}

// O row qrow = acc / l in bf16 (rows past T skipped).
__device__ __forceinline__ void store_rows(const SoftmaxState& st, uint16_t* __restrict__ obase,
                                           int64_t so_t, int qrow, int T, int half) {
  const float inv = 1.f / xhalf_sum(st.l);
  if (qrow >= T) return;
  uint16_t* orow = obase + static_cast<int64_t>(qrow) * so_t;
  // the two lanes of a row swap halves so each writes 16 contiguous bytes
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int ip = 0; ip < 2; ++ip) {
      uint32_t w[2][2];
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int i = 2 * ip + u;
        w[u][0] = pack_bf16x2(st.acc[dt][4 * i] * inv, st.acc[dt][4 * i + 1] * inv);
        w[u][1] = pack_bf16x2(st.acc[dt][4 * i + 2] * inv, st.acc[dt][4 * i + 3] * inv);
      }
      uint32_t y[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const uint32_t x = half ? w[0][e] : w[1][e];
        const auto r = __builtin_amdgcn_permlane32_swap(x, x, false, false);
        y[e] = half ? r[0] : r[1];
      }
      const uint4 v = half ? make_uint4(y[0], y[1], w[1][0], w[1][1]) : make_uint4(w[0][0], w[0][1], y[0], y[1]);
      *reinterpret_cast<uint4*>(orow + 32 * dt + 16 * ip + 8 * half) = v;
    }
}

// ------------------------------------------------------------ argument checks
inline int check_fwd_common(const void* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                            const void* kc, const void* vc, int64_t npad, const int32_t* counts,
                            const uint32_t* mask, int64_t B, int64_t T,
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
  SOLATTN_REQUIRE(q && kc && vc && counts && mask && o, SOLATTN_EINVAL, "%s: null pointer", what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(q) % 16 == 0 && sq_b % 8 == 0 && sq_t % 8 == 0 &&
                      sq_h % 8 == 0,
                  SOLATTN_EINVAL, "%s: q must be 16-byte aligned with strides multiple of 8", what);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(kc) % 16 == 0 && reinterpret_cast<uintptr_t>(vc) % 16 == 0,
                  SOLATTN_EINVAL, "%s: kc/vc must be 16-byte aligned", what);
  // store_rows writes each output row as 16-byte stores
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(o) % 16 == 0 && so_b % 8 == 0 && so_t % 8 == 0 &&
                      so_h % 8 == 0,
                  SOLATTN_EINVAL, "%s: o must be 16-byte aligned with strides multiple of 8", what);
  return 0;
}

inline int check_fwd_args(const void* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const void* k,
                          int64_t sk_b, int64_t sk_t, int64_t sk_h, const void* v, int64_t sv_b,
                          int64_t sv_t, int64_t sv_h, const void* kc, const void* vc, int64_t npad,
                          const int32_t* counts, const uint32_t* mask,
                          int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, const void* o,
                          int64_t so_b, int64_t so_t, int64_t so_h, const char* what) {
  if (int rc = check_fwd_common(q, sq_b, sq_t, sq_h, kc, vc, npad, counts, mask, B, T, H, D,
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
