// Row gather for the Morton token permutation and its inverse:
//   dst[b, t, :] = src[b, index[t], :]
// HBM-bound copy: every workgroup moves a run of whole rows in 16-byte lanes,
// so each wave issues fully coalesced 1 KiB loads and stores. Replaces the
// torch index_select calls of /root/reference/_morton.py:113,128,148 and
// /root/reference/_morton_h3.py:193,217.
#include <algorithm>

#include "common.hpp"

namespace solattn {

constexpr int kReorderThreads = 256;
constexpr int kReorderChunksPerThread = 8;  // 16-byte chunks in flight per thread

__global__ void __launch_bounds__(kReorderThreads)
reorder_rows_kernel(const char* __restrict__ src, int64_t src_stride_b, int64_t src_stride_row,
                    char* __restrict__ dst, int64_t dst_stride_b, int64_t dst_stride_row,
                    const int64_t* __restrict__ index, int64_t src_rows, uint32_t rows,
                    uint32_t chunks_per_row, uint32_t rows_per_wg) {
  const uint32_t b = blockIdx.y;
  const uint32_t r0 = blockIdx.x * rows_per_wg;
  const uint32_t nrows = min(rows_per_wg, rows - r0);
  const uint32_t total = nrows * chunks_per_row;
  const char* sb = src + static_cast<int64_t>(b) * src_stride_b;
  char* db = dst + static_cast<int64_t>(b) * dst_stride_b;
  for (uint32_t base = 0; base < total; base += kReorderThreads * kReorderChunksPerThread) {
    uint4 v[kReorderChunksPerThread];
    uint32_t row[kReorderChunksPerThread], col[kReorderChunksPerThread];
#pragma unroll
    for (int u = 0; u < kReorderChunksPerThread; ++u) {
      uint32_t e = base + u * kReorderThreads + threadIdx.x;
      row[u] = e / chunks_per_row;
      col[u] = e - row[u] * chunks_per_row;
      v[u] = make_uint4(0u, 0u, 0u, 0u);
      if (e < total) {
        int64_t srow = index[r0 + row[u]];
        // An index outside the source rows yields a zero row instead of a fault.
        if (srow >= 0 && srow < src_rows)
          v[u] = *reinterpret_cast<const uint4*>(sb + srow * src_stride_row + col[u] * 16u);
      }
    }
#pragma unroll
    for (int u = 0; u < kReorderChunksPerThread; ++u) {
      uint32_t e = base + u * kReorderThreads + threadIdx.x;
      if (e < total)
        *reinterpret_cast<uint4*>(db + static_cast<int64_t>(r0 + row[u]) * dst_stride_row +
                                  col[u] * 16u) = v[u];
    }
  }
}

// ------------------------------------------------------------- head padding
// dst[b, t, h, :] = (src[b, t, h, 0:din], zeros) for a dense [B, T, H, dout]
// destination (pad, din < dout), or the reverse slice src[..., 0:dout] into a
// strided destination (unpad, din > dout): the one-call pipelines run head
// dims below 128 on the D = 128 kernels. Zero channels add exact zeros to
// every dot product and pooled sum, so routing, codes and outputs are those of
// the unpadded problem. One thread moves 8 bf16 (16 bytes).
__global__ void __launch_bounds__(256)
pad_heads_kernel(const uint16_t* __restrict__ src, int64_t s_b, int64_t s_t, int64_t s_h,
                 uint16_t* __restrict__ dst, int64_t d_b, int64_t d_t, int64_t d_h, int64_t T,
                 int H, int din, int dout, int64_t rows) {
  const int per_row = dout / 8;
  const int64_t e = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (e >= rows * per_row) return;
  const int64_t row = e / per_row;
  const int c8 = static_cast<int>(e - row * per_row) * 8;
  const int64_t h = row % H, bt = row / H, t = bt % T, b = bt / T;
  uint4 v = make_uint4(0u, 0u, 0u, 0u);
  if (c8 < din) v = *reinterpret_cast<const uint4*>(src + b * s_b + t * s_t + h * s_h + c8);
  *reinterpret_cast<uint4*>(dst + b * d_b + t * d_t + h * d_h + c8) = v;
}

int pad_heads(const uint16_t* src, int64_t s_b, int64_t s_t, int64_t s_h, uint16_t* dst,
              int64_t d_b, int64_t d_t, int64_t d_h, int64_t B, int64_t T, int64_t H, int64_t din,
              int64_t dout, hipStream_t stream) {
  SOLATTN_REQUIRE(src && dst && din % 8 == 0 && dout % 8 == 0, SOLATTN_EINVAL,
                  "pad_heads: bad arguments");
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(src) % 16 == 0 && reinterpret_cast<uintptr_t>(dst) % 16 == 0 &&
                      s_b % 8 == 0 && s_t % 8 == 0 && s_h % 8 == 0 && d_b % 8 == 0 &&
                      d_t % 8 == 0 && d_h % 8 == 0,
                  SOLATTN_EINVAL, "pad_heads: rows must be 16-byte aligned");
  const int64_t rows = B * T * H;
  const int64_t work = rows * (dout / 8);
  SOLATTN_REQUIRE(cdiv(work, 256) < (1ll << 31), SOLATTN_EUNSUPPORTED, "pad_heads: too large");
  hipLaunchKernelGGL(pad_heads_kernel, dim3(static_cast<uint32_t>(cdiv(work, 256))), dim3(256), 0,
                     stream, src, s_b, s_t, s_h, dst, d_b, d_t, d_h, T, static_cast<int>(H),
                     static_cast<int>(din), static_cast<int>(dout), rows);
  return check_launch("pad_heads");
}

}  // namespace solattn

using namespace solattn;

extern "C" int solattn_reorder_rows(const void* src, int64_t src_rows, int64_t src_stride_b_bytes,
                                    int64_t src_stride_row_bytes, void* dst,
                                    int64_t dst_stride_b_bytes, int64_t dst_stride_row_bytes,
                                    int64_t batch, int64_t rows, int64_t row_bytes,
                                    const int64_t* index, solattn_stream_t stream) {
  clear_error();
  if (batch == 0 || rows == 0) return SOLATTN_OK;
  SOLATTN_REQUIRE(src && dst && index, SOLATTN_EINVAL, "reorder: null pointer");
  SOLATTN_REQUIRE(batch > 0 && rows > 0 && src_rows > 0 && row_bytes > 0, SOLATTN_EINVAL,
                  "reorder: bad sizes batch=%lld rows=%lld src_rows=%lld row_bytes=%lld",
                  (long long)batch, (long long)rows, (long long)src_rows, (long long)row_bytes);
  SOLATTN_REQUIRE(row_bytes % 16 == 0 && src_stride_row_bytes % 16 == 0 &&
                      dst_stride_row_bytes % 16 == 0 && src_stride_b_bytes % 16 == 0 &&
                      dst_stride_b_bytes % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(src) % 16 == 0 &&
                      reinterpret_cast<uintptr_t>(dst) % 16 == 0,
                  SOLATTN_EINVAL, "reorder: rows, strides and bases must be 16-byte aligned");
  SOLATTN_REQUIRE(rows < (1ll << 31) && row_bytes / 16 < (1ll << 24) && batch <= 65535,
                  SOLATTN_EUNSUPPORTED, "reorder: sizes beyond the 32-bit index range");
  const uint32_t cpr = static_cast<uint32_t>(row_bytes / 16);
  // About 4096 chunks (64 KiB) per workgroup, at least one row.
  uint32_t rows_per_wg = static_cast<uint32_t>(std::max<int64_t>(1, 4096 / cpr));
  rows_per_wg = std::min<uint32_t>(rows_per_wg, static_cast<uint32_t>(rows));
  SOLATTN_REQUIRE(static_cast<uint64_t>(rows_per_wg) * cpr < (1ull << 31), SOLATTN_EUNSUPPORTED,
                  "reorder: row too long");
  dim3 grid(static_cast<uint32_t>(cdiv(rows, rows_per_wg)), static_cast<uint32_t>(batch));
  hipLaunchKernelGGL(reorder_rows_kernel, grid, dim3(kReorderThreads), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const char*>(src),
                     src_stride_b_bytes, src_stride_row_bytes, static_cast<char*>(dst),
                     dst_stride_b_bytes, dst_stride_row_bytes, index, src_rows,
                     static_cast<uint32_t>(rows), cpr, rows_per_wg);
  return check_launch("reorder_rows");
}

