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

// Head dims the one-call pipelines take: multiples of 8 up to the kernels'
// 128; smaller heads are zero-padded to 128 in the workspace.
constexpr int64_t kKernelD = 128;
inline bool pipeline_head_dim_ok(int64_t D) { return D >= 8 && D <= kKernelD && D % 8 == 0; }

// Carves the pipeline's intermediates out of one workspace.
struct Layout {
  int64_t NT, npad, W, TP;
  int64_t kc, vc, qbar, kc_mean, kc_var, thr, counts, mask;   // byte offsets
  int64_t vamax, vscale, qi, qs, ki, ks, vi;                          // INT8 only
  int64_t qp, kp, vp, op;  // zero-padded [B, T, H, 128] q, k, v, o (head dims < 128)
  bool padded;
  int64_t total;
  Layout(int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, bool int8) {
    const int64_t Dk = kKernelD;
    NT = cdiv(T, block);
    npad = cdiv(NT, 64) * 64;
    W = cdiv(NT, 32);
    TP = T;
    padded = D != Dk;
    int64_t off = 0;
    auto take = [&](int64_t bytes) {
      const int64_t at = off;
      off += cdiv(bytes, 256) * 256;
      return at;
    };
    kc = take(B * npad * H * Dk * 2);
    vc = take(B * npad * H * Dk * 2);
    qbar = take(B * H * NT * Dk * 4);
    kc_mean = take(B * H * Dk * 4);
    kc_var = take(B * H * Dk * 4);
    thr = take(B * NT * H * 4);
    counts = take(B * H * NT * 4);
    mask = take(B * H * NT * W * 4);
    vamax = vscale = qi = qs = ki = ks = vi = -1;
    if (int8) {
      vamax = take(B * NT * H * Dk * 4);
      vscale = take(B * H * Dk * 4);
      qi = take(B * TP * H * Dk);
      qs = take(B * TP * H * 4);
      ki = take(B * TP * H * Dk);
      ks = take(B * TP * H * 4);
      vi = take(B * TP * H * Dk);
    }
    qp = kp = vp = op = -1;
    if (padded) {
      qp = take(B * T * H * Dk * 2);
      kp = take(B * T * H * Dk * 2);
      vp = take(B * T * H * Dk * 2);
      op = take(B * T * H * Dk * 2);
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

extern "C" int solattn_abi_version(void) { return (2 << 16) | 1; }

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

// One call's operands: BTHD q, k, v (element strides), the output and the
// problem sizes and routing parameters.
struct Call {
  const uint16_t* q; int64_t sq_b, sq_t, sq_h;
  const uint16_t* k; int64_t sk_b, sk_t, sk_h;
  const uint16_t* v; int64_t sv_b, sv_t, sv_h;
  uint16_t* o; int64_t so_b, so_t, so_h;
  int64_t B, T, H, D, block;
  float scale, tau;
  int64_t skv_lo, skv_hi, sq_lo, sq_hi;
};

// Runs fn on the call as the D = 128 kernels see it: unchanged when D is 128,
// else on zero-padded copies of q, k, v in the workspace with the output
// sliced back into the caller's o afterwards (zero channels add exact zeros
// to every dot product and sum).
template <typename F>
int with_kernel_head_dim(const Layout& L, void* ws, const Call& c, hipStream_t s, F&& fn) {
  if (!L.padded) return fn(c);
  const int64_t Dk = kKernelD, st = c.H * Dk, sb = c.T * st;
  Call p = c;
  uint16_t* qp = at<uint16_t>(ws, L.qp);
  uint16_t* kp = at<uint16_t>(ws, L.kp);
  uint16_t* vp = at<uint16_t>(ws, L.vp);
  uint16_t* op = at<uint16_t>(ws, L.op);
  int rc = pad_heads(c.q, c.sq_b, c.sq_t, c.sq_h, qp, sb, st, Dk, c.B, c.T, c.H, c.D, Dk, s);
  if (!rc) rc = pad_heads(c.k, c.sk_b, c.sk_t, c.sk_h, kp, sb, st, Dk, c.B, c.T, c.H, c.D, Dk, s);
  if (!rc) rc = pad_heads(c.v, c.sv_b, c.sv_t, c.sv_h, vp, sb, st, Dk, c.B, c.T, c.H, c.D, Dk, s);
  if (rc) return rc;
  p.q = qp; p.k = kp; p.v = vp; p.o = op;
  p.sq_b = p.sk_b = p.sv_b = p.so_b = sb;
  p.sq_t = p.sk_t = p.sv_t = p.so_t = st;
  p.sq_h = p.sk_h = p.sv_h = p.so_h = Dk;
  p.D = Dk;
  if ((rc = fn(p))) return rc;
  return pad_heads(op, sb, st, Dk, c.o, c.so_b, c.so_t, c.so_h, c.B, c.T, c.H, Dk, c.D, s);
}

// pool -> moments -> route -> fwd_bf16 over the intermediates of `L` carved
// out of ws (256-byte aligned, at least L.total bytes; nothing in it needs to
// start zeroed: every byte a later stage reads is written by an earlier one).
int run_bf16_pipeline(const Layout& L, void* ws, const Call& call, solattn_stream_t stream) {
  return with_kernel_head_dim(L, ws, call, reinterpret_cast<hipStream_t>(stream), [&](const Call& c) {
    int rc = solattn_pool(c.q, c.sq_b, c.sq_t, c.sq_h, c.k, c.sk_b, c.sk_t, c.sk_h, c.v, c.sv_b,
                          c.sv_t, c.sv_h, c.B, c.T, c.H, c.D, c.block, at<uint16_t>(ws, L.kc),
                          at<uint16_t>(ws, L.vc), L.npad, at<float>(ws, L.qbar), nullptr, stream);
    if (rc) return rc;
    rc = solattn_moments(at<uint16_t>(ws, L.kc), L.npad, c.B, L.NT, c.H, c.D, 0,
                         at<float>(ws, L.kc_mean), at<float>(ws, L.kc_var), nullptr, nullptr, stream);
    if (rc) return rc;
    rc = solattn_route(at<float>(ws, L.qbar), at<uint16_t>(ws, L.kc), L.npad,
                       at<float>(ws, L.kc_mean), at<float>(ws, L.kc_var), c.B, c.T, c.H, c.D,
                       c.block, c.scale, c.tau, 0, c.skv_lo, c.skv_hi, c.sq_lo, c.sq_hi,
                       at<float>(ws, L.thr), at<int32_t>(ws, L.counts), at<uint32_t>(ws, L.mask), stream);
    if (rc) return rc;
    return solattn_fwd_bf16(c.q, c.sq_b, c.sq_t, c.sq_h, c.k, c.sk_b, c.sk_t, c.sk_h, c.v, c.sv_b,
                            c.sv_t, c.sv_h, at<uint16_t>(ws, L.kc), at<uint16_t>(ws, L.vc), L.npad,
                            at<int32_t>(ws, L.counts), at<uint32_t>(ws, L.mask), c.B, c.T, c.H, c.D, c.block, c.scale, c.o,
                            c.so_b, c.so_t, c.so_h, stream);
  });
}

// pool -> moments(centre) -> route(mode 1) -> quant(q, k smoothed, v) -> fwd_int8.
int run_int8_pipeline(const Layout& L, void* ws, const Call& call, int int8_pv,
                      solattn_stream_t stream, int qk_block = 0) {
  hipStream_t hs = reinterpret_cast<hipStream_t>(stream);
  return with_kernel_head_dim(L, ws, call, hs, [&](const Call& c) {
    float* vamax = int8_pv ? at<float>(ws, L.vamax) : nullptr;
    float* vscale = int8_pv ? at<float>(ws, L.vscale) : nullptr;
    // Two passes: the pooling pass also quantises Q per token (the only tensor
    // whose codes need no statistic over the whole head), so Q is read once;
    // per block the quantisation pass takes Q with K. (The single-read
    // preparation, solattn_prep_int8, reads K and V once too, but its heads
    // run one after another through two barriers and it measured slower at
    // every shape: 0.66 ms more per call at config 2, 0.08 ms at config 1.)
    int rc = pool_checked(c.q, c.sq_b, c.sq_t, c.sq_h, c.k, c.sk_b, c.sk_t, c.sk_h, c.v, c.sv_b,
                          c.sv_t, c.sv_h, c.B, c.T, c.H, c.D, c.block, at<uint16_t>(ws, L.kc),
                          at<uint16_t>(ws, L.vc), L.npad, at<float>(ws, L.qbar), vamax,
                          qk_block ? nullptr : at<int8_t>(ws, L.qi),
                          qk_block ? nullptr : at<float>(ws, L.qs), L.TP, hs);
    if (rc) return rc;
    rc = solattn_moments(at<uint16_t>(ws, L.kc), L.npad, c.B, L.NT, c.H, c.D, 1,
                         at<float>(ws, L.kc_mean), at<float>(ws, L.kc_var), vamax, vscale, stream);
    if (rc) return rc;
    rc = solattn_route(at<float>(ws, L.qbar), at<uint16_t>(ws, L.kc), L.npad, nullptr,
                       at<float>(ws, L.kc_var), c.B, c.T, c.H, c.D, c.block, c.scale, c.tau, 1,
                       c.skv_lo, c.skv_hi, c.sq_lo, c.sq_hi, at<float>(ws, L.thr),
                       at<int32_t>(ws, L.counts), at<uint32_t>(ws, L.mask), stream);
    if (rc) return rc;
    rc = quant_qkv(qk_block ? c.q : nullptr, c.sq_b, c.sq_t, c.sq_h, c.k, c.sk_b, c.sk_t, c.sk_h,
                   c.v, c.sv_b, c.sv_t, c.sv_h, c.B, c.T, c.H, c.D, at<float>(ws, L.kc_mean),
                   vscale, at<int8_t>(ws, L.qi), at<float>(ws, L.qs), at<int8_t>(ws, L.ki),
                   at<float>(ws, L.ks), int8_pv ? at<int8_t>(ws, L.vi) : nullptr, L.TP, hs,
                   qk_block, /*ks_head_major=*/1);
    if (rc) return rc;
    // per block, every 64-key tile of K shares one scale: the forward folds it
    // into the tile's score factor. K's scales are kept head-major here, so a
    // tile's 64 scales are one contiguous 256-byte read.
    return fwd_int8(c.q, c.sq_b, c.sq_t, c.sq_h, at<int8_t>(ws, L.qi), at<float>(ws, L.qs),
                    at<int8_t>(ws, L.ki), at<float>(ws, L.ks),
                    int8_pv ? at<int8_t>(ws, L.vi) : nullptr, vscale, c.v, c.sv_b, c.sv_t, c.sv_h,
                    L.TP, at<uint16_t>(ws, L.kc), at<uint16_t>(ws, L.vc), L.npad,
                    at<int32_t>(ws, L.counts), at<uint32_t>(ws, L.mask),
                    c.B, c.T, c.H, c.D, c.block, c.scale, int8_pv, c.o, c.so_b, c.so_t, c.so_h,
                    stream, qk_block != 0, /*ks_head_major=*/true);
  });
}

int check_pipeline(int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, const char* what) {
  SOLATTN_REQUIRE(B > 0 && T > 0 && H > 0 && block > 0, SOLATTN_EINVAL, "%s: bad sizes", what);
  SOLATTN_REQUIRE(pipeline_head_dim_ok(D), SOLATTN_EUNSUPPORTED,
                  "%s: head_dim %lld (multiples of 8 up to 128)", what, (long long)D);
  return 0;
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
  if (int rc = check_pipeline(B, T, H, D, block, "sol_attn")) return rc;
  const Layout L(B, T, H, D, block, false);
  SOLATTN_REQUIRE(workspace && workspace_bytes >= L.total, SOLATTN_ESIZE,
                  "sol_attn: workspace %lld < %lld bytes", (long long)workspace_bytes,
                  (long long)L.total);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, SOLATTN_EINVAL,
                  "sol_attn: workspace must be 256-byte aligned");
  const Call c{q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, o, so_b, so_t, so_h,
               B, T, H, D, block, scale, tau, sink_kv_lo, sink_kv_hi, sink_q_lo, sink_q_hi};
  return run_bf16_pipeline(L, workspace, c, stream);
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
  if (int rc = check_pipeline(B, T, H, D, block, "sol_attn_noalloc")) return rc;
  const Layout L(B, T, H, D, block, false);
  SOLATTN_REQUIRE(L.total <= SOLATTN_NOALLOC_SCRATCH_BYTES, SOLATTN_ESIZE,
                  "sol_attn_noalloc: B=%lld T=%lld H=%lld block=%lld needs %lld bytes of "
                  "intermediates, more than the %lld-byte scratch; use solattn_sol_attn with a "
                  "workspace",
                  (long long)B, (long long)T, (long long)H, (long long)block, (long long)L.total,
                  (long long)SOLATTN_NOALLOC_SCRATCH_BYTES);
  void* ws = nullptr;
  if (int rc = scratch_for_current_device(&ws)) return rc;
  const Call c{q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, o, so_b, so_t, so_h,
               B, T, H, D, block, scale, tau, sink_kv_lo, sink_kv_hi, sink_q_lo, sink_q_hi};
  return run_bf16_pipeline(L, ws, c, stream);
}

#define SOLATTN_INT8_CALL_PARAMS                                                               \
  const uint16_t *q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t *k, int64_t sk_b,   \
      int64_t sk_t, int64_t sk_h, const uint16_t *v, int64_t sv_b, int64_t sv_t, int64_t sv_h,    \
      int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, float scale, float tau,          \
      int64_t sink_kv_lo, int64_t sink_kv_hi, int64_t sink_q_lo, int64_t sink_q_hi, int int8_pv,  \
      void *workspace, int64_t workspace_bytes, uint16_t *o, int64_t so_b, int64_t so_t,          \
      int64_t so_h, solattn_stream_t stream

namespace {

int sol_attn_int8_call(SOLATTN_INT8_CALL_PARAMS, int qk_block) {
  clear_error();
  if (int rc = check_pipeline(B, T, H, D, block, "sol_attn_int8")) return rc;
  SOLATTN_REQUIRE(int8_pv >= SOLATTN_PV_BF16 && int8_pv <= SOLATTN_PV_INT8_RUNNING, SOLATTN_EINVAL,
                  "sol_attn_int8: int8_pv %d is not a SOLATTN_PV_* mode", int8_pv);
  const Layout L(B, T, H, D, block, true);
  SOLATTN_REQUIRE(workspace && workspace_bytes >= L.total, SOLATTN_ESIZE,
                  "sol_attn_int8: workspace %lld < %lld bytes", (long long)workspace_bytes,
                  (long long)L.total);
  SOLATTN_REQUIRE(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, SOLATTN_EINVAL,
                  "sol_attn_int8: workspace must be 256-byte aligned");
  const Call c{q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, o, so_b, so_t, so_h,
               B, T, H, D, block, scale, tau, sink_kv_lo, sink_kv_hi, sink_q_lo, sink_q_hi};
  return run_int8_pipeline(L, workspace, c, int8_pv, stream, qk_block);
}

}  // namespace

extern "C" int solattn_sol_attn_int8(SOLATTN_INT8_CALL_PARAMS) {
  return sol_attn_int8_call(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B, T, H,
                            D, block, scale, tau, sink_kv_lo, sink_kv_hi, sink_q_lo, sink_q_hi,
                            int8_pv, workspace, workspace_bytes, o, so_b, so_t, so_h, stream, 0);
}

extern "C" int solattn_sol_attn_int8_qblock(SOLATTN_INT8_CALL_PARAMS) {
  return sol_attn_int8_call(q, sq_b, sq_t, sq_h, k, sk_b, sk_t, sk_h, v, sv_b, sv_t, sv_h, B, T, H,
                            D, block, scale, tau, sink_kv_lo, sink_kv_hi, sink_q_lo, sink_q_hi,
                            int8_pv, workspace, workspace_bytes, o, so_b, so_t, so_h, stream, 1);
}
