// C ABI glue: thread-local error messages, the host-side Morton permutation,
// and the one-call pipelines (pool -> moments -> route -> [quant] -> forward)
// over a caller-owned workspace, plus the BF16 pipeline over a fixed
// per-device scratch array for callers that cannot allocate. The library
// never calls an allocator.
#include <stdarg.h>
#include <stdio.h>

#include <algorithm>
#include <mutex>
#include <numeric>
#include <vector>

#include "common.hpp"

namespace solattn {

namespace {
thread_local char g_error[512] = "";
}

int set_error(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(g_error, sizeof(g_error), fmt, ap);
  va_end(ap);
  return code;
}

void clear_error() { g_error[0] = '\0'; }

int check_launch(const char* what) {
  const hipError_t e = hipGetLastError();
  if (e != hipSuccess) return set_error(SOLATTN_ELAUNCH, "%s: launch failed: %s", what, hipGetErrorString(e));
  return SOLATTN_OK;
}

// Spreads the low 21 bits of v two bits apart (bit i -> bit 3i), the
// coordinate interleave of /root/reference/_morton.py:56-63.
uint64_t spread3(uint64_t v) {
  uint64_t out = 0;
  for (int i = 0; i < 21; ++i) out |= ((v >> i) & 1ull) << (3 * i);
  return out;
}

// Carves the pipeline's intermediates out of one workspace.
struct Layout {
  int64_t NT, npad, W, TP;
  int64_t kc, vc, qbar, kc_mean, kc_var, thr, counts, lists, mask;   // byte offsets
  int64_t vamax, vscale, qi, qs, ki, ks, vi;                          // INT8 only
  int64_t total;
  Layout(int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, bool int8) {
    NT = cdiv(T, block);
    npad = cdiv(NT, 64) * 64;
    W = cdiv(NT, 32);
    TP = T;
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
      const int64_t at = off;
      off += cdiv(bytes, 256) * 256;
      return at;
    };
    kc = take(B * npad * H * D * 2);
    vc = take(B * npad * H * D * 2);
    qbar = take(B * H * NT * D * 4);
    kc_mean = take(B * H * D * 4);
    kc_var = take(B * H * D * 4);
    thr = take(B * NT * H * 4);
    counts = take(B * H * NT * 4);
    lists = take(B * H * NT * NT * 2);
    mask = take(B * H * NT * W * 4);
    vamax = vscale = qi = qs = ki = ks = vi = -1;
    if (int8) {
      vamax = take(B * NT * H * D * 4);
      vscale = take(B * H * D * 4);
      qi = take(B * TP * H * D);
      qs = take(B * TP * H * 4);
      ki = take(B * TP * H * D);
      ks = take(B * TP * H * 4);
      vi = take(B * TP * H * D);
    }
    total = off;
  }
};

template <typename P>
P* at(void* ws, int64_t off) {
  return reinterpret_cast<P*>(static_cast<char*>(ws) + off);
}

}  // namespace solattn

using namespace solattn;

extern "C" const char* solattn_last_error(void) { return g_error; }

extern "C" int solattn_abi_version(void) { return (1 << 16) | 0; }

extern "C" int solattn_morton_perm(int64_t frames, int64_t height, int64_t width, int curve,
                                   int64_t roll, int64_t* perm, int64_t* inverse) {
  clear_error();
  SOLATTN_REQUIRE(frames > 0 && height > 0 && width > 0, SOLATTN_EINVAL, "morton: empty grid");
  SOLATTN_REQUIRE(frames < (1 << 21) && height < (1 << 21) && width < (1 << 21), SOLATTN_EINVAL,
                  "morton: grid dims must be < 2^21");
  SOLATTN_REQUIRE(curve == SOLATTN_CURVE_3D || curve == SOLATTN_CURVE_2D_FRAME, SOLATTN_EINVAL,
                  "morton: unknown curve %d", curve);
  SOLATTN_REQUIRE(perm && inverse, SOLATTN_EINVAL, "morton: null output");
  const int64_t n = frames * height * width, area = height * width;
  std::vector<uint64_t> code(n);
  for (int64_t lin = 0; lin < n; ++lin) {
    const uint64_t z = lin / area, rem = lin % area, y = rem / width, x = rem % width;
    code[lin] = curve == SOLATTN_CURVE_2D_FRAME ? ((z << 42) | spread3(x) | (spread3(y) << 1))
                                                : (spread3(x) | (spread3(y) << 1) | (spread3(z) << 2));
  }
  std::vector<int64_t> order(n);
  std::iota(order.begin(), order.end(), 0);
  std::sort(order.begin(), order.end(), [&](int64_t a, int64_t b) { return code[a] < code[b]; });
  const int64_t r = ((roll % n) + n) % n;  // torch.roll: out[(i + r) % n] = in[i]
  for (int64_t i = 0; i < n; ++i) perm[(i + r) % n] = order[i];
  for (int64_t i = 0; i < n; ++i) inverse[perm[i]] = i;
  return SOLATTN_OK;
}

extern "C" int64_t solattn_sol_attn_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D,
                                                    int64_t block, int int8) {
  if (B <= 0 || T <= 0 || H <= 0 || D <= 0 || block <= 0) return 0;
  return Layout(B, T, H, D, block, int8 != 0).total;
}

namespace solattn {
namespace {

// pool -> moments -> route -> fwd_bf16 over the intermediates of `L` carved
// out of ws (256-byte aligned, at least L.total bytes; nothing in it needs to
// start zeroed: every byte a later stage reads is written by an earlier one).
int run_bf16_pipeline(const Layout& L, void* ws, const uint16_t* q, int64_t sq_b, int64_t sq_t,
                      int64_t sq_h, const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                      const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                      int64_t T, int64_t H, int64_t D, int64_t block, float scale, float tau,
                      int64_t sink_kv_lo, int64_t sink_kv_hi, int64_t sink_q_lo,
                      int64_t sink_q_hi, uint16_t* o, int64_t so_b, int64_t so_t, int64_t so_h,
                      solattn_stream_t stream) {
  int rc = solattn_pool(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B, T, H, D,
                        block, at<uint16_t>(ws, L.kc), at<uint16_t>(ws, L.vc), L.npad,
                        at<float>(ws, L.qbar), nullptr, stream);
  if (rc) return rc;
  rc = solattn_moments(at<uint16_t>(ws, L.kc), L.npad, B, L.NT, H, D, 0, at<float>(ws, L.kc_mean),
                       at<float>(ws, L.kc_var), nullptr, nullptr, stream);
  if (rc) return rc;
  rc = solattn_route(at<float>(ws, L.qbar), at<uint16_t>(ws, L.kc), L.npad, at<float>(ws, L.kc_mean),
                     at<float>(ws, L.kc_var), B, T, H, D, block, scale, tau, 0, sink_kv_lo,
                     sink_kv_hi, sink_q_lo, sink_q_hi, at<float>(ws, L.thr), at<int32_t>(ws, L.counts),
                     at<int16_t>(ws, L.lists), at<uint32_t>(ws, L.mask), stream);
  if (rc) return rc;
  return solattn_fwd_bf16(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h,
                          at<uint16_t>(ws, L.kc), at<uint16_t>(ws, L.vc), L.npad,
                          at<int32_t>(ws, L.counts), at<int16_t>(ws, L.lists),
                          at<uint32_t>(ws, L.mask), B, T, H, D, block, scale, o, so_b, so_t, so_h,
                          stream);
}

// The allocation-free pipeline's intermediates: one fixed array per device,
// loaded with the code object. In host code `scratch` names a host-side
// stand-in, not device memory; only the address hipGetSymbolAddress returns
// for the current device is ever handed to a kernel.
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices] = {};

}  // namespace
}  // namespace solattn

static __device__ __align__(256) unsigned char scratch[SOLATTN_NOALLOC_SCRATCH_BYTES];

namespace solattn {
namespace {

// This device's copy of `scratch`, looked up once per device (with that
// device current) and kept for the life of the process.
int scratch_for_current_device(void** out) {
  int dev = -1;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess)
    return set_error(SOLATTN_ELAUNCH, "sol_attn_noalloc: hipGetDevice: %s", hipGetErrorString(e));
  SOLATTN_REQUIRE(dev >= 0 && dev < kMaxScratchDevices, SOLATTN_EUNSUPPORTED,
                  "sol_attn_noalloc: device %d beyond the %d supported", dev, kMaxScratchDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    const hipError_t r = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (r != hipSuccess || p == nullptr)
      return set_error(SOLATTN_ELAUNCH, "sol_attn_noalloc: hipGetSymbolAddress(scratch): %s",
                       hipGetErrorString(r));
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return SOLATTN_OK;
}

}  // namespace
}  // namespace solattn

extern "C" int solattn_sol_attn(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                                const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                                float scale, float tau, int64_t sink_kv_lo, int64_t sink_kv_hi,
                                int64_t sink_q_lo, int64_t sink_q_hi, void* workspace,
                                int64_t workspace_bytes, uint16_t* o, int64_t so_b, int64_t so_t,
                                int64_t so_h, solattn_stream_t stream) {
  clear_error();
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && block > 0, SOLATTN_EINVAL, "sol_attn: bad sizes");
  const Layout L(B, T, H, D, block, false);
  SOLATTN_REQUIRE(workspace && workspace_bytes >= L.total, SOLATTN_ESIZE,
                  "sol_attn: workspace %lld < %lld bytes", (long long)workspace_bytes,
                  (long long)L.total);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, SOLATTN_EINVAL,
                  "sol_attn: workspace must be 256-byte aligned");
  return run_bf16_pipeline(L, workspace, q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t,
                           sv_h, B, T, H, D, block, scale, tau, sink_kv_lo, sink_kv_hi, sink_q_lo,
                           sink_q_hi, o, so_b, so_t, so_h, stream);
}

extern "C" int solattn_sol_attn_noalloc(const uint16_t* q, int64_t sq_b, int64_t sq_t,
                                        int64_t sq_h, const uint16_t* k, int64_t sk_b,
                                        int64_t sk_t, int64_t sk_h, const uint16_t* v,
                                        int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                                        int64_t T, int64_t H, int64_t D, int64_t block,
                                        float scale, float tau, int64_t sink_kv_lo,
                                        int64_t sink_kv_hi, int64_t sink_q_lo, int64_t sink_q_hi,
                                        uint16_t* o, int64_t so_b, int64_t so_t, int64_t so_h,
                                        solattn_stream_t stream) {
  clear_error();
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && block > 0, SOLATTN_EINVAL,
                  "sol_attn_noalloc: bad sizes");
  const Layout L(B, T, H, D, block, false);
  SOLATTN_REQUIRE(L.total <= SOLATTN_NOALLOC_SCRATCH_BYTES, SOLATTN_ESIZE,
                  "sol_attn_noalloc: B=%lld T=%lld H=%lld block=%lld needs %lld bytes of "
                  "intermediates, more than the %lld-byte scratch; use solattn_sol_attn with a "
                  "workspace",
                  (long long)B, (long long)T, (long long)H, (long long)block, (long long)L.total,
                  (long long)SOLATTN_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws)) return rc;
  return run_bf16_pipeline(L, ws, q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h,
                           B, T, H, D, block, scale, tau, sink_kv_lo, sink_kv_hi, sink_q_lo,
                           sink_q_hi, o, so_b, so_t, so_h, stream);
}

extern "C" int solattn_sol_attn_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                     const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                                     const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                     int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                                     float scale, float tau, int64_t sink_kv_lo,
                                     int64_t sink_kv_hi, int64_t sink_q_lo, int64_t sink_q_hi,
                                     int int8_pv, void* workspace, int64_t workspace_bytes,
                                     uint16_t* o, int64_t so_b, int64_t so_t, int64_t so_h,
                                     solattn_stream_t stream) {
  clear_error();
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && block > 0, SOLATTN_EINVAL, "sol_attn_int8: bad sizes");
  const Layout L(B, T, H, D, block, true);
  SOLATTN_REQUIRE(workspace && workspace_bytes >= L.total, SOLATTN_ESIZE,
                  "sol_attn_int8: workspace %lld < %lld bytes", (long long)workspace_bytes,
                  (long long)L.total);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, SOLATTN_EINVAL,
                  "sol_attn_int8: workspace must be 256-byte aligned");
  void* ws = workspace;
  float* vamax = int8_pv ? at<float>(ws, L.vamax) : nullptr;
  float* vscale = int8_pv ? at<float>(ws, L.vscale) : nullptr;
  int rc = solattn_pool(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B, T, H, D,
                        block, at<uint16_t>(ws, L.kc), at<uint16_t>(ws, L.vc), L.npad,
                        at<float>(ws, L.qbar), vamax, stream);
  if (rc) return rc;
  rc = solattn_moments(at<uint16_t>(ws, L.kc), L.npad, B, L.NT, H, D, 1, at<float>(ws, L.kc_mean),
                       at<float>(ws, L.kc_var), vamax, vscale, stream);
  if (rc) return rc;
  rc = solattn_route(at<float>(ws, L.qbar), at<uint16_t>(ws, L.kc), L.npad, nullptr,
                     at<float>(ws, L.kc_var), B, T, H, D, block, scale, tau, 1, sink_kv_lo,
                     sink_kv_hi, sink_q_lo, sink_q_hi, at<float>(ws, L.thr), at<int32_t>(ws, L.counts),
                     at<int16_t>(ws, L.lists), at<uint32_t>(ws, L.mask), stream);
  if (rc) return rc;
  rc = quant_qkv(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B, T, H, D,
                 at<float>(ws, L.kc_mean), vscale, at<int8_t>(ws, L.qi), at<float>(ws, L.qs),
                 at<int8_t>(ws, L.ki), at<float>(ws, L.ks), int8_pv ? at<int8_t>(ws, L.vi) : nullptr,
                 L.TP, reinterpret_cast<hipStream_t>(stream));
  if (rc) return rc;
  return solattn_fwd_int8(q, sq_b, sq_t, sq_h, at<int8_t>(ws, L.qi), at<float>(ws, L.qs),
                          at<int8_t>(ws, L.ki), at<float>(ws, L.ks),
                          int8_pv ? at<int8_t>(ws, L.vi) : nullptr, vscale, v, sv_b, sv_t, sv_h,
                          L.TP, at<uint16_t>(ws, L.kc), at<uint16_t>(ws, L.vc), L.npad,
                          at<int32_t>(ws, L.counts), at<int16_t>(ws, L.lists),
                          at<uint32_t>(ws, L.mask), B, T, H, D, block, scale, int8_pv, o, so_b,
                          so_t, so_h, stream);
}
