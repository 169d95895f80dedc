// Hardware ceilings of gfx950 that bound the forward kernels, measured with
// one stand-alone program (no library code): sustained bf16 MFMA rate, LDS
// read rates in the forward's own operand patterns, and MFMA fed by one LDS
// operand per instruction. The shader clock is measured in the kernels
// themselves: s_memtime (shader clock) against s_memrealtime (100 MHz).
//
// Launch shape: 512 workgroups of 256 threads (two per CU, two waves per SIMD),
// as the block-128 forward. Every LDS address is masked into the kernel's
// 64 KiB buffer; every global store writes index blockIdx.x < grid.
//
// Build and run (gfx950):
//   hipcc --offload-arch=gfx950 -O3 -Xclang -target-feature -Xclang -packed-fp32-ops \
//       hw_ceilings.hip -o /tmp/hw_ceilings && /tmp/hw_ceilings
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <vector>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef short v4i16 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) v4i16 lds_v4;
typedef __attribute__((address_space(3))) u32x2 lds_u2;
typedef __attribute__((address_space(3))) u32x4 lds_u4;
typedef __attribute__((address_space(3))) bf16x8 lds_bf16x8;

struct Stamp {
  uint64_t t0, t1, r0, r1;  // shader clock and 100 MHz real-time counter
};

constexpr int kGrid = 512;
constexpr int kThreads = 256;

// Independent accumulation chains of v_mfma_f32_32x32x16_bf16.
__global__ void __launch_bounds__(kThreads) mfma_loop(int iters, float* out, Stamp* st) {
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(threadIdx.x * 1e-3f + i);
    b[i] = (__bf16)(i * 0.5f);
  }
  f32x16 acc[4] = {};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[c] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[c], 0, 0, 0);
  }
  float s = 0.f;
  for (int c = 0; c < 4; ++c)
    for (int i = 0; i < 16; ++i) s += acc[c][i];
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (s == 12345.f) out[blockIdx.x] = s;
  if (threadIdx.x == 0) st[blockIdx.x] = Stamp{t0, t1, r0, r1};
}

// LDS byte address of a __shared__ array.
__device__ inline uint32_t lds_base(uint32_t* p) {
  return static_cast<uint32_t>(reinterpret_cast<uintptr_t>((__attribute__((address_space(3))) uint32_t*)p));
}

// Operand lane addresses of the forward (one 16 KiB tile of 64 rows x 256 B).
__device__ inline uint32_t k_lane(uint32_t tile, int col, int half) {
  return tile + col * 256 + 16 * (half ^ (col & 15));
}
__device__ inline uint32_t v_lane(uint32_t tile, int lane) {
  const int g = lane >> 4, sl = lane & 15;
  const int row0 = 4 * (g >> 1) + (sl >> 2);
  const int cp = 2 * (g & 1) + ((sl & 3) >> 1);
  return tile + row0 * 256 + 64 * (row0 & 3) + 16 * cp + 8 * (sl & 1);
}

// LDS reads over four 16 KiB tiles, 16 KiB per wave per iteration.
// MODE 0: ds_read_b64, lanes contiguous. MODE 1: K operands, ds_read_b128 at
// (k_lane ^ (cc << 5)) + 8192 m. MODE 2: V operands, two ds_read_b64_tr_b16
// at (v_lane ^ (dt << 6)) + 4096 ks (+2048).
template <int MODE>
__global__ void __launch_bounds__(kThreads) lds_loop(int iters, uint32_t* out, Stamp* st) {
  __shared__ __attribute__((aligned(256))) uint32_t buf[16384];
  for (int i = threadIdx.x; i < 16384; i += kThreads) buf[i] = i * 2654435761u;
  __syncthreads();
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t b0 = lds_base(buf);
  uint32_t x = 0;
  for (int it = 0; it < iters; ++it) {
    const uint32_t tile = b0 + (((it + w) & 3) << 14);
    if (MODE == 0) {
#pragma unroll
      for (int k = 0; k < 32; ++k) {
        const u32x2 v = *(lds_u2*)(uintptr_t)(tile + lane * 8 + k * 512);
        x ^= v.x ^ v.y;
      }
    } else if (MODE == 1) {
      const uint32_t kl = k_lane(tile, lane & 31, lane >> 5);
#pragma unroll
      for (int m = 0; m < 2; ++m)
#pragma unroll
        for (int cc = 0; cc < 8; ++cc) {
          const u32x4 v = *(lds_u4*)(uintptr_t)((kl ^ static_cast<uint32_t>(cc << 5)) + m * 8192);
          x ^= v.x ^ v.y ^ v.z ^ v.w;
        }
    } else {
      const uint32_t vl = v_lane(tile, lane);
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) {
          const uint32_t a = (vl ^ static_cast<uint32_t>(dt << 6)) + ks * 4096;
          const v4i16 lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(uintptr_t)a);
          const v4i16 hi = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_v4*)(uintptr_t)(a + 2048));
          x ^= static_cast<uint32_t>(lo[0] ^ lo[1] ^ lo[2] ^ lo[3] ^ hi[0] ^ hi[1] ^ hi[2] ^ hi[3]);
        }
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (x == 0x12345678u) out[blockIdx.x] = x;
  if (threadIdx.x == 0) st[blockIdx.x] = Stamp{t0, t1, r0, r1};
}

// MFMA whose A operand comes from LDS (K operand pattern, one ds_read_b128 =
// 1 KiB per wave per MFMA), the ratio of a 32-row wave in the forward.
__global__ void __launch_bounds__(kThreads) mfma_lds_loop(int iters, float* out, Stamp* st) {
  __shared__ __attribute__((aligned(256))) uint32_t buf[16384];
  for (int i = threadIdx.x; i < 16384; i += kThreads) buf[i] = 0x3f803f80u;
  __syncthreads();
  const uint64_t t0 = __builtin_amdgcn_s_memtime(), r0 = __builtin_amdgcn_s_memrealtime();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const uint32_t b0 = lds_base(buf);
  bf16x8 b;
  for (int i = 0; i < 8; ++i) b[i] = (__bf16)(i * 0.5f);
  f32x16 acc[4] = {};
  for (int it = 0; it < iters; ++it) {
    const uint32_t kl = k_lane(b0 + (((it + w) & 3) << 14), lane & 31, lane >> 5);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      const bf16x8 a = *(lds_bf16x8*)(uintptr_t)((kl ^ static_cast<uint32_t>((i & 7) << 5)) + (i >> 3) * 8192);
      acc[i & 3] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc[i & 3], 0, 0, 0);
    }
  }
  float s = 0.f;
  for (int c = 0; c < 4; ++c)
    for (int i = 0; i < 16; ++i) s += acc[c][i];
  const uint64_t t1 = __builtin_amdgcn_s_memtime(), r1 = __builtin_amdgcn_s_memrealtime();
  if (s == 12345.f) out[blockIdx.x] = s;
  if (threadIdx.x == 0) st[blockIdx.x] = Stamp{t0, t1, r0, r1};
}

#define CK(x)                                                                        \
  do {                                                                               \
    hipError_t e = (x);                                                              \
    if (e != hipSuccess) {                                                           \
      fprintf(stderr, "HIP error %s at line %d\n", hipGetErrorString(e), __LINE__); \
      exit(1);                                                                       \
    }                                                                                \
  } while (0)

// Times one launch (after one warm-up launch); prints the rate in `unit`, the
// shader clock during the kernel and the rate per CU per clock.
template <typename F>
void run(const char* name, F launch, double work_per_wg, const char* unit, double unit_scale,
         Stamp* st) {
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  launch();
  CK(hipDeviceSynchronize());
  CK(hipEventRecord(e0));
  launch();
  CK(hipEventRecord(e1));
  CK(hipEventSynchronize(e1));
  float ms;
  CK(hipEventElapsedTime(&ms, e0, e1));
  std::vector<Stamp> h(kGrid);
  CK(hipMemcpy(h.data(), st, kGrid * sizeof(Stamp), hipMemcpyDeviceToHost));
  double cyc = 0, rt = 0;
  for (const Stamp& s : h) {
    cyc += double(s.t1 - s.t0);
    rt += double(s.r1 - s.r0);
  }
  const double ghz = cyc / (rt / 100e6) / 1e9;
  const double total = work_per_wg * kGrid;
  printf("| %-34s | %8.3f | %9.1f %-7s | %5.2f | %7.1f |\n", name, ms, total / (ms * 1e-3) / unit_scale,
         unit, ghz, total / 256.0 / (ms * 1e-3 * ghz * 1e9));
  CK(hipEventDestroy(e0));
  CK(hipEventDestroy(e1));
}

int main() {
  Stamp* st;
  float* out;
  CK(hipMalloc(&st, kGrid * sizeof(Stamp)));
  CK(hipMalloc(&out, kGrid * sizeof(float)));
  const int it_m = 20000, it_l = 20000;
  const double waves = kThreads / 64;
  printf("| kernel | ms | rate | GHz | per CU per clock |\n|---|---:|---:|---:|---:|\n");
  for (int rep = 0; rep < 2; ++rep) {
    run("bf16 MFMA 32x32x16, 4 chains", [&] { hipLaunchKernelGGL(mfma_loop, dim3(kGrid), dim3(kThreads), 0, 0, it_m, out, st); },
        waves * 4 * it_m * 32768.0, "TFLOP/s", 1e12, st);
    run("LDS ds_read_b64, contiguous", [&] { hipLaunchKernelGGL(lds_loop<0>, dim3(kGrid), dim3(kThreads), 0, 0, it_l, (uint32_t*)out, st); },
        waves * 16384.0 * it_l, "TB/s", 1e12, st);
    run("LDS ds_read_b128, K operand pattern", [&] { hipLaunchKernelGGL(lds_loop<1>, dim3(kGrid), dim3(kThreads), 0, 0, it_l, (uint32_t*)out, st); },
        waves * 16384.0 * it_l, "TB/s", 1e12, st);
    run("LDS ds_read_b64_tr_b16, V pattern", [&] { hipLaunchKernelGGL(lds_loop<2>, dim3(kGrid), dim3(kThreads), 0, 0, it_l, (uint32_t*)out, st); },
        waves * 16384.0 * it_l, "TB/s", 1e12, st);
    run("MFMA + 1 KiB LDS operand each", [&] { hipLaunchKernelGGL(mfma_lds_loop, dim3(kGrid), dim3(kThreads), 0, 0, it_m / 4, out, st); },
        waves * 16 * (it_m / 4) * 32768.0, "TFLOP/s", 1e12, st);
  }
  CK(hipFree(st));
  CK(hipFree(out));
  return 0;
}
