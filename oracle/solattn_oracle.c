/*
 * CPU oracle for the Sol-Attn sparse attention path -- TEST INFRASTRUCTURE.
 *
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * this library, and only as the checker (or the timed CPU baseline). It is never
 * on the product path: the package fails loudly when its HIP library is missing.
 *
 * Each function restates the reference's algorithm (file:line cited) with the
 * operation order fixed by the arithmetic contract in include/solattn.h, so the
 * HIP kernels can be compared bit for bit:
 *   - pooled sums: sixteen fp32 partials over rows r = g (mod 16), ascending,
 *     combined by the pairwise tree of tree16() below;
 *   - moments: 8 partials over blocks j = g (mod 8), ascending, combined as
 *     a fixed tree; no FMA;
 *   - dot products for thresholds and routing: fmaf chains over d ascending.
 * Build: see oracle/Makefile (gcc -O2 -ffp-contract=off, no fast-math).
 *
 * Parity pins (tests/test_oracle_*.py): Morton against brute-force bit loops and
 * textbook orders; pooling/threshold/routing against float64 closed forms and
 * hand-built band/sink cases; quant against hand-picked known answers.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

/* ------------------------------------------------------------------ bf16 */
static inline float bf2f(uint16_t h) {
  uint32_t u = (uint32_t)h << 16;
  float f;
  memcpy(&f, &u, 4);
  return f;
}

/* Round-to-nearest-even fp32 -> bf16 (NaN kept quiet). */
static inline uint16_t f2bf(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40);
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

uint16_t or_f2bf(float f) { return f2bf(f); }
float or_bf2f(uint16_t h) { return bf2f(h); }

/* ---------------------------------------------------------------- Morton --
 * /root/reference/_morton.py:49-71: decompose linear -> (z=t, y, x), spread
 * each coordinate's 21 low bits two apart, interleave; 2d_frame puts the frame
 * index above bit 42. perm = argsort(code) (codes are unique, so the order is
 * unique), inverse = argsort(perm). roll: /root/reference/_morton_h3.py:50-53. */
static uint64_t part1by2(uint64_t v) {
  v &= 0x1FFFFFull;
  v = (v | (v << 32)) & 0x1F00000000FFFFull;
  v = (v | (v << 16)) & 0x1F0000FF0000FFull;
  v = (v | (v << 8)) & 0x100F00F00F00F00Full;
  v = (v | (v << 4)) & 0x10C30C30C30C30C3ull;
  v = (v | (v << 2)) & 0x1249249249249249ull;
  return v;
}

static const uint64_t* g_codes;
static int cmp_code(const void* a, const void* b) {
  uint64_t ca = g_codes[*(const int64_t*)a], cb = g_codes[*(const int64_t*)b];
  return ca < cb ? -1 : (ca > cb ? 1 : 0);
}

int or_morton_perm(int64_t frames, int64_t height, int64_t width, int curve, int64_t roll,
                   int64_t* perm, int64_t* inverse) {
  int64_t n = frames * height * width;
  if (n <= 0) return 0;
  uint64_t* code = (uint64_t*)malloc(sizeof(uint64_t) * (size_t)n);
  int64_t* tmp = (int64_t*)malloc(sizeof(int64_t) * (size_t)n);
  if (!code || !tmp) { free(code); free(tmp); return -1; }
  int64_t area = height * width;
  for (int64_t lin = 0; lin < n; ++lin) {
    uint64_t z = (uint64_t)(lin / area), rem = (uint64_t)(lin % area);
    uint64_t y = rem / (uint64_t)width, x = rem % (uint64_t)width;
    code[lin] = curve == 1 ? ((z << 42) | part1by2(x) | (part1by2(y) << 1))
                           : (part1by2(x) | (part1by2(y) << 1) | (part1by2(z) << 2));
    tmp[lin] = lin;
  }
  g_codes = code;
  qsort(tmp, (size_t)n, sizeof(int64_t), cmp_code);
  int64_t r = ((roll % n) + n) % n; /* torch.roll: out[(i + r) % n] = in[i] */
  for (int64_t i = 0; i < n; ++i) perm[(i + r) % n] = tmp[i];
  for (int64_t i = 0; i < n; ++i) inverse[perm[i]] = i;
  free(code);
  free(tmp);
  return 0;
}

/* ------------------------------------------------------------------ pool --
 * /root/reference/_preprocess.py:49-57 (kc = sum/len), :100 (vc = sum),
 * :106-113 (per-block |v| max), :140-149 (q centroid = sum/len).
 * x: bf16 BTHD with element strides; rows t >= T read as 0. For every
 * (head, channel) sixteen partials take rows r = g (mod 16) in ascending order
 * and combine by tree16; rows are streamed so the loop is cache-friendly. */
static inline float tree16(const float* p, int64_t stride) {
  float a[8];
  for (int i = 0; i < 8; ++i) a[i] = p[(2 * i) * stride] + p[(2 * i + 1) * stride];
  return ((a[0] + a[1]) + (a[2] + a[3])) + ((a[4] + a[5]) + (a[6] + a[7]));
}

static void pool_one(const uint16_t* x, int64_t s_b, int64_t s_t, int64_t s_h, int64_t b,
                     int64_t t0, int64_t T, int64_t H, int64_t D, int64_t block, float* part,
                     float* amax, float* out_sum) {
  int64_t HD = H * D;
  for (int64_t e = 0; e < 16 * HD; ++e) part[e] = 0.f;
  if (amax)
    for (int64_t e = 0; e < HD; ++e) amax[e] = 0.f;
  for (int64_t r = 0; r < block; ++r) {
    int64_t t = t0 + r;
    float* p = part + (r & 15) * HD;
    for (int64_t h = 0; h < H; ++h) {
      const uint16_t* row = t < T ? x + b * s_b + t * s_t + h * s_h : NULL;
      for (int64_t d = 0; d < D; ++d) {
        float val = row ? bf2f(row[d]) : 0.f;
        p[h * D + d] = p[h * D + d] + val;
        if (amax) {
          float a = fabsf(val);
          if (a > amax[h * D + d]) amax[h * D + d] = a;
        }
      }
    }
  }
  for (int64_t e = 0; e < HD; ++e) out_sum[e] = tree16(part + e, HD);
}

void or_pool(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h, const uint16_t* k,
             int64_t sk_b, int64_t sk_t, int64_t sk_h, const uint16_t* v, int64_t sv_b,
             int64_t sv_t, int64_t sv_h, int64_t B, int64_t T, int64_t H, int64_t D,
             int64_t block, uint16_t* kc, uint16_t* vc, int64_t npad, float* qbar,
             float* vamax_part) {
  int64_t NT = (T + block - 1) / block;
  int64_t HD = H * D;
#pragma omp parallel
  {
    float* part = (float*)malloc(sizeof(float) * (size_t)(16 * HD));
    float* sk = (float*)malloc(sizeof(float) * (size_t)HD);
    float* sv = (float*)malloc(sizeof(float) * (size_t)HD);
    float* sq = (float*)malloc(sizeof(float) * (size_t)HD);
    float* am = (float*)malloc(sizeof(float) * (size_t)HD);
#pragma omp for collapse(2) schedule(static)
    for (int64_t b = 0; b < B; ++b)
      for (int64_t j = 0; j < NT; ++j) {
        int64_t t0 = j * block;
        int64_t len = T - t0 < block ? T - t0 : block;
        float flen = (float)len;
        pool_one(k, sk_b, sk_t, sk_h, b, t0, T, H, D, block, part, NULL, sk);
        pool_one(v, sv_b, sv_t, sv_h, b, t0, T, H, D, block, part, am, sv);
        pool_one(q, sq_b, sq_t, sq_h, b, t0, T, H, D, block, part, NULL, sq);
        for (int64_t h = 0; h < H; ++h)
          for (int64_t d = 0; d < D; ++d) {
            int64_t e = h * D + d;
            int64_t o = ((b * npad + j) * H + h) * D + d;
            kc[o] = f2bf(sk[e] / flen);
            vc[o] = f2bf(sv[e]);
            qbar[((b * H + h) * NT + j) * D + d] = sq[e] / flen;
            if (vamax_part) vamax_part[((b * NT + j) * H + h) * D + d] = am[e];
          }
      }
    free(part);
    free(sk);
    free(sv);
    free(sq);
    free(am);
  }
}

/* Sums over blocks use 8 partials (blocks j = g mod 8, ascending) combined
 * ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)). */
static inline float tree8(const float* p) {
  return ((p[0] + p[1]) + (p[2] + p[3])) + ((p[4] + p[5]) + (p[6] + p[7]));
}

/* --------------------------------------------------------------- moments --
 * BF16: /root/reference/_preprocess.py:241-243 (mean and population variance
 * over valid blocks). INT8: /root/reference/_fused_prep.py:77-81 (centre kc by
 * its own mean, store bf16, variance of the stored values). V scale:
 * /root/reference/_fused_quant.py:102-105 and _preprocess.py:221-223. */
void or_moments(uint16_t* kc, int64_t npad, int64_t B, int64_t NT, int64_t H, int64_t D,
                int centre, float* kc_mean, float* kc_var, const float* vamax_part,
                float* vscale) {
  float fnt = (float)NT;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t d = 0; d < D; ++d) {
        float s[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int64_t j = 0; j < NT; ++j)
          s[j & 7] = s[j & 7] + bf2f(kc[((b * npad + j) * H + h) * D + d]);
        float mean = tree8(s) / fnt;
        float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
        for (int64_t j = 0; j < NT; ++j) {
          uint16_t* e = &kc[((b * npad + j) * H + h) * D + d];
          float x;
          if (centre) {
            *e = f2bf(bf2f(*e) - mean);
            x = bf2f(*e);
          } else {
            x = bf2f(*e) - mean;
          }
          acc[j & 7] = acc[j & 7] + x * x;
        }
        kc_mean[(b * H + h) * D + d] = mean;
        kc_var[(b * H + h) * D + d] = tree8(acc) / fnt;
        if (vamax_part && vscale) {
          float m = 0.f;
          for (int64_t j = 0; j < NT; ++j) {
            float a = vamax_part[((b * NT + j) * H + h) * D + d];
            if (a > m) m = a;
          }
          /* torch's GPU div by a scalar multiplies by the fp32 reciprocal, so
           * absmax.div(127.0) is absmax * (1/127)f. */
          float sc = m * (1.0f / 127.0f);
          vscale[(b * H + h) * D + d] = sc < 1e-8f ? 1e-8f : sc;
        }
      }
}

/* ----------------------------------------------------------------- route --
 * Threshold: BF16 /root/reference/_preprocess.py:149-163; INT8
 * /root/reference/_fused_prep.py:50-59. Routing rule: the forward's
 * /root/reference/_tri_fwd.py:279-286 (R = sum_r (q_r . kc_j) * c / len_i,
 * restated as c * (qbar_i . kc_j)); exact = q_in_sink ? valid : routed. */
void or_threshold(const float* qbar, const float* kc_mean, const float* kc_var, int64_t B,
                  int64_t NT, int64_t H, int64_t D, float scale, float tau, int mode,
                  float* thr) {
  float c = scale * 1.4426950408889634f;
  float c2 = c * c;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t i = 0; i < NT; ++i) {
        const float* qb = qbar + ((b * H + h) * NT + i) * D;
        const float* mu_k = kc_mean + (b * H + h) * D;
        const float* var_k = kc_var + (b * H + h) * D;
        float mu = 0.f, var = 0.f;
        for (int64_t d = 0; d < D; ++d) {
          if (mode == 0) mu = fmaf(qb[d], mu_k[d], mu);
          var = fmaf(qb[d] * qb[d], var_k[d], var);
        }
        float t;
        if (mode == 0) {
          mu = mu * c;
          var = var * c2;
          float sd = sqrtf(fmaxf(var, 0.f) + 1e-6f);
          t = mu + tau * sd;
        } else {
          var = var * c2;
          t = tau * sqrtf(var + 1e-6f);
        }
        thr[(b * NT + i) * H + h] = t;
      }
}

float or_route_score(const float* qb, const uint16_t* kcj, int64_t D, float scale) {
  float c = scale * 1.4426950408889634f;
  float acc = 0.f;
  for (int64_t d = 0; d < D; ++d) acc = fmaf(qb[d], bf2f(kcj[d]), acc);
  return acc * c;
}

void or_route(const float* qbar, const uint16_t* kc, int64_t npad, const float* thr,
              int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, float scale,
              int64_t sink_kv_lo, int64_t sink_kv_hi, int64_t sink_q_lo, int64_t sink_q_hi,
              int32_t* counts, int16_t* lists, uint32_t* mask, float* scores) {
  int64_t NT = (T + block - 1) / block;
  int64_t W = (NT + 31) / 32;
#pragma omp parallel for collapse(3) schedule(dynamic, 4)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t h = 0; h < H; ++h)
      for (int64_t i = 0; i < NT; ++i) {
        const float* qb = qbar + ((b * H + h) * NT + i) * D;
        float t = thr[(b * NT + i) * H + h];
        int q_in_sink = i >= sink_q_lo && i < sink_q_hi;
        int64_t row = (b * H + h) * NT + i;
        uint32_t* mrow = mask + row * W;
        for (int64_t w = 0; w < W; ++w) mrow[w] = 0;
        int32_t n = 0;
        for (int64_t j = 0; j < NT; ++j) {
          float r = or_route_score(qb, kc + ((b * npad + j) * H + h) * D, D, scale);
          if (scores) scores[row * NT + j] = r;
          int64_t dij = i > j ? i - j : j - i;
          int routed = (r > t) || dij <= 1 || (j >= sink_kv_lo && j < sink_kv_hi);
          int exact = q_in_sink ? 1 : routed;
          if (exact) {
            lists[row * NT + n] = (int16_t)j;
            ++n;
            mrow[j >> 5] |= 1u << (j & 31);
          }
        }
        counts[row] = n;
      }
}

/* ----------------------------------------------------------------- quant --
 * Per token: /root/reference/_fused_quant.py:25-42 (K, optional smoothing
 * mean, round-then-clamp) and /root/reference/_fused_prep.py:43-48 (Q,
 * clamp-then-round; identical codes). */
static inline int8_t round_half_away_clamp(float val) {
  float r = val >= 0.f ? truncf(val + 0.5f) : truncf(val - 0.5f);
  if (r < -127.f) r = -127.f;
  if (r > 127.f) r = 127.f;
  return (int8_t)r;
}

void or_quant_rows(const uint16_t* x, int64_t sx_b, int64_t sx_t, int64_t sx_h, int64_t B,
                   int64_t T, int64_t H, int64_t D, const float* mean, int8_t* xi, float* xs,
                   int64_t TP) {
  if (D > 4096) return;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t h = 0; h < H; ++h) {
        float y[4096];
        float amax = 0.f;
        for (int64_t d = 0; d < D; ++d) {
          float val = bf2f(x[b * sx_b + t * sx_t + h * sx_h + d]);
          if (mean) val = val - mean[(b * H + h) * D + d];
          y[d] = val;
          float a = fabsf(val);
          if (a > amax) amax = a;
        }
        float s = amax / 127.0f;
        float ss = s > 1e-8f ? s : 1e-8f;
        int64_t o = ((b * TP + t) * H + h) * D;
        for (int64_t d = 0; d < D; ++d) xi[o + d] = round_half_away_clamp(y[d] / ss);
        xs[(b * TP + t) * H + h] = ss;
      }
}

/* Per block of QB tokens (BASELINE config 3's "Q/K quantised per 128-token
 * block ... fp32 scales (symmetric, absmax)"; the reference itself quantises
 * per token): one scale per (b, block, h) from the |max| over the block's
 * tokens and channels, the same code rule as per token, and the block's scale
 * written for every token of the block. */
void or_quant_rows_blocked(const uint16_t* x, int64_t sx_b, int64_t sx_t, int64_t sx_h,
                           int64_t B, int64_t T, int64_t H, int64_t D, const float* mean,
                           int8_t* xi, float* xs, int64_t TP, int64_t QB) {
  if (QB <= 0) return;
  const int64_t NB = (T + QB - 1) / QB;
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t j = 0; j < NB; ++j)
      for (int64_t h = 0; h < H; ++h) {
        const int64_t t0 = j * QB, t1 = t0 + QB < T ? t0 + QB : T;
        float amax = 0.f;
        for (int64_t t = t0; t < t1; ++t)
          for (int64_t d = 0; d < D; ++d) {
            float val = bf2f(x[b * sx_b + t * sx_t + h * sx_h + d]);
            if (mean) val = val - mean[(b * H + h) * D + d];
            float a = fabsf(val);
            if (a > amax) amax = a;
          }
        float s = amax / 127.0f;
        float ss = s > 1e-8f ? s : 1e-8f;
        for (int64_t t = t0; t < t1; ++t) {
          int64_t o = ((b * TP + t) * H + h) * D;
          for (int64_t d = 0; d < D; ++d) {
            float val = bf2f(x[b * sx_b + t * sx_t + h * sx_h + d]);
            if (mean) val = val - mean[(b * H + h) * D + d];
            xi[o + d] = round_half_away_clamp(val / ss);
          }
          xs[(b * TP + t) * H + h] = ss;
        }
      }
}

/* Per channel V: /root/reference/_fused_quant.py:77-88. */
void or_quant_v(const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                int64_t T, int64_t H, int64_t D, const float* vscale, int8_t* vi, int64_t TP) {
#pragma omp parallel for collapse(2) schedule(static)
  for (int64_t b = 0; b < B; ++b)
    for (int64_t t = 0; t < T; ++t)
      for (int64_t h = 0; h < H; ++h)
        for (int64_t d = 0; d < D; ++d) {
          float val = bf2f(v[b * sv_b + t * sv_t + h * sv_h + d]);
          vi[((b * TP + t) * H + h) * D + d] =
              round_half_away_clamp(val / vscale[(b * H + h) * D + d]);
        }
}

/* ------------------------------------------------------------ test helper --
 * The INT8 kernels form a per-token scale fl(amax / 127) without a division,
 * as fma(fma(-q0, 127, a), c, q0) with q0 = a * c and c = fl(1/127). Counts the
 * non-negative finite floats a (bit patterns start, start + step, ... below
 * stop) for which that differs from the IEEE quotient. */
uint64_t or_div127_mismatches(uint32_t start, uint32_t stop, uint32_t step) {
  const float c = 1.0f / 127.0f;
  uint64_t bad = 0;
  if (stop > 0x7f800000u) stop = 0x7f800000u;
  for (uint64_t u = start; u < stop; u += step) {
    uint32_t bits = (uint32_t)u;
    float a;
    memcpy(&a, &bits, sizeof a);
    const float q0 = a * c;
    const float q1 = fmaf(fmaf(-q0, 127.0f, a), c, q0);
    if (q1 != a / 127.0f) ++bad;
  }
  return bad;
}
