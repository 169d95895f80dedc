/*
 * solattn.h -- C ABI of libsolattn.so, the gfx950 (MI355X) implementation of
 * Sol-Attn's sparse attention path.
 *
 * Conventions shared by every entry point:
 *  - Device pointers are plain pointers into HBM; "bf16" buffers hold bfloat16
 *    bit patterns (uint16_t). Strides are in ELEMENTS unless a name ends in
 *    _bytes. Inputs q/k/v are BTHD ([batch, tokens, heads, head_dim]) with only
 *    the last dim required to be contiguous; every other buffer is a dense
 *    allocation in the layout written next to it.
 *  - block is the routing block size in tokens (64 or 128); NT = ceil(T/block)
 *    query/key blocks; npad is the block dim of kc/vc (>= NT, zero padded).
 *  - Every function returns 0 on success or a negative SOLATTN_E* code and
 *    records a message readable with solattn_last_error() (thread-local).
 *  - The library never allocates device memory and never synchronises: every
 *    launch goes on the hipStream_t passed in (NULL = the null stream).
 *  - head_dim must be 128 for the per-kernel entry points (the reference
 *    node's only eligible head size, /root/reference/__init__.py:41,178); the
 *    one-call pipelines (solattn_sol_attn*) also take head dims that are
 *    multiples of 8 below 128 (the reference kernels' D = 64 configs,
 *    /root/reference/_tri_fwd.py:209), running them zero-padded to 128 in the
 *    workspace: zero channels add exact zeros to every dot product and sum,
 *    so routing, codes and outputs are those of the unpadded problem, at the
 *    cost of a D = 128 call.
 *
 * Arithmetic contract (the CPU oracle restates the same operation order, so
 * pooled keys, thresholds, routing masks and INT8 codes are bit-exact):
 *  - pooled sums: for each (block, channel) sixteen fp32 partial sums p_g over
 *    the block's rows r = g (mod 16) taken in ascending order (rows past T add
 *    0.0f), combined pairwise as ((((p0+p1)+(p2+p3))+((p4+p5)+(p6+p7))) +
 *    (((p8+p9)+(p10+p11))+((p12+p13)+(p14+p15)))).
 *  - kc = bf16_rne(sum / len); vc = bf16_rne(sum); qbar = sum / len (fp32).
 *  - moments: 8 fp32 partials over blocks j = g (mod 8), ascending, combined
 *    ((p0+p1)+(p2+p3)) + ((p4+p5)+(p6+p7)); no FMA.
 *  - routing score R[i][j] = (fmaf chain over d of qbar_i[d] * kc_j[d]) * c,
 *    c = scale * 1.4426950408889634f; thresholds as documented per function.
 */
#ifndef SOLATTN_H
#define SOLATTN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* solattn_stream_t; /* == hipStream_t */

enum {
  SOLATTN_OK = 0,
  SOLATTN_EINVAL = -1,    /* bad argument (shape, stride, null pointer) */
  SOLATTN_EUNSUPPORTED = -2, /* valid but not implemented (e.g. head_dim != 128) */
  SOLATTN_ELAUNCH = -3,   /* HIP launch error */
  SOLATTN_ESIZE = -4      /* buffer too small */
};

enum { SOLATTN_CURVE_3D = 0, SOLATTN_CURVE_2D_FRAME = 1 };

/* int8_pv of the INT8 entry points: how P.V runs (solattn_fwd_int8). */
enum {
  SOLATTN_PV_BF16 = 0,         /* bf16 P against bf16 v */
  SOLATTN_PV_INT8 = 1,         /* int8 codes against each routed block's row max */
  SOLATTN_PV_INT8_RUNNING = 2  /* int8 codes against the row's running max */
};

/* Message for the last failing call on this thread ("" if none). */
const char* solattn_last_error(void);
/* ABI version: (major << 16) | minor. */
int solattn_abi_version(void);

/* ---------------------------------------------------------------- Morton --
 * Host function (no device work). Z-order permutation of a frames x height x
 * width latent grid laid out frame-major, then row-major, and its inverse.
 * curve SOLATTN_CURVE_3D interleaves x, y, t bits; SOLATTN_CURVE_2D_FRAME keeps
 * the frame index as the most significant key. roll != 0 rotates perm by roll
 * places (torch.roll semantics) before the inverse is taken.
 * perm/inverse: host int64 arrays of frames*height*width entries.
 * Replaces: morton_perm, /root/reference/_morton.py:35-73, and the span roll of
 * _perm_for, /root/reference/_morton_h3.py:42-61. */
int solattn_morton_perm(int64_t frames, int64_t height, int64_t width, int curve,
                        int64_t roll, int64_t* perm, int64_t* inverse);

/* --------------------------------------------------------------- reorder --
 * Row gather: dst[b, t, :] = src[b, index[t], :] for t < rows, b < batch.
 * A row is row_bytes contiguous bytes (row_bytes % 16 == 0, 16-byte aligned
 * rows). index: device int64 [rows], each entry in [0, src_rows).
 * Replaces: the torch index_select / fancy-index gathers of the Morton hooks,
 * /root/reference/_morton.py:113,128,148 and /root/reference/_morton_h3.py:193,217. */
int solattn_reorder_rows(const void* src, int64_t src_rows, int64_t src_stride_b_bytes,
                         int64_t src_stride_row_bytes, void* dst, int64_t dst_stride_b_bytes,
                         int64_t dst_stride_row_bytes, int64_t batch, int64_t rows,
                         int64_t row_bytes, const int64_t* index, solattn_stream_t stream);

/* ------------------------------------------------------------------ pool --
 * One pass over q, k and v per (batch, block, head):
 *   kc[b, j, h, :] = bf16_rne(sum_k / len_j)      kc, vc: bf16 [B, npad, H, D]
 *   vc[b, j, h, :] = bf16_rne(sum_v)              (rows j >= NT are not written)
 *   qbar[b, h, j, :] = sum_q / len_j              qbar: fp32 [B, H, NT, D]
 *   vamax_part[b, j, h, :] = max_r |v|            fp32 [B, NT, H, D], may be NULL
 * Token strides must lie in [0, 2^26) elements and T <= 65535 * 128
 * (SOLATTN_EUNSUPPORTED otherwise).
 * Replaces: _reduce_kc_kernel / _reduce_vc_kernel / _reduce_kv,
 * /root/reference/_preprocess.py:23-113,172-224, and the Q centroid of
 * _diag_threshold_kernel (:144-149) / _q_quant_threshold_kernel
 * (/root/reference/_fused_prep.py:16-59). */
int solattn_pool(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                 const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                 const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                 int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                 uint16_t* kc, uint16_t* vc, int64_t npad, float* qbar,
                 float* vamax_part, solattn_stream_t stream);

/* --------------------------------------------------------------- moments --
 * Per (b, h, d) over blocks j < NT, in ascending j:
 *   mean = (sum_j kc) / NT
 *   centre == 0 (BF16 path, /root/reference/_preprocess.py:241-243):
 *     var = (sum_j (kc - mean)^2) / NT
 *   centre == 1 (INT8 path, /root/reference/_fused_prep.py:77-81):
 *     kc[b, j, h, d] = bf16_rne(kc - mean) (in place); var = (sum_j kc'^2) / NT
 * kc_mean, kc_var: fp32 [B, H, D].
 * If vamax_part != NULL also vscale[b, h, d] = max(max_j vamax_part * (1/127)f, 1e-8)
 * (/root/reference/_fused_quant.py:102-105: torch divides by a scalar as a
 * multiply by its fp32 reciprocal). kc and vamax_part must be 16-byte aligned;
 * with vamax_part, H < 32768 (SOLATTN_EUNSUPPORTED otherwise). */
int solattn_moments(uint16_t* kc, int64_t npad, int64_t B, int64_t NT, int64_t H,
                    int64_t D, int centre, float* kc_mean, float* kc_var,
                    const float* vamax_part, float* vscale, solattn_stream_t stream);

/* ----------------------------------------------------------------- route --
 * Thresholds, routing decisions and per-query-block exact-block masks.
 *   mode 0 (BF16, /root/reference/_preprocess.py:150-163):
 *     mu  = (fmaf chain qbar*kc_mean) * c
 *     var = (fmaf chain (qbar*qbar)*kc_var) * (c*c)
 *     thr = mu + tau * sqrtf(fmaxf(var, 0) + 1e-6f)
 *   mode 1 (INT8, /root/reference/_fused_prep.py:50-59, kc already centred):
 *     thr = tau * sqrtf(var + 1e-6f)
 *   R[i][j] = (fmaf chain qbar_i*kc_j) * c
 *   exact(i, j) = i in [sink_q_lo, sink_q_hi) ? 1
 *               : R > thr || |i - j| <= 1 || j in [sink_kv_lo, sink_kv_hi)
 *   (the forward's rule, /root/reference/_tri_fwd.py:279-286).
 * Outputs: thr fp32 [B, NT, H]; counts int32 [B, H, NT] (exact blocks per
 * query block); mask uint32 [B, H, NT, ceil(NT/32)] (bit j%32 of word j/32 =
 * exact; bits j >= NT are 0). The reference keeps no list either: it re-derives
 * the decisions in every forward program. */
int solattn_route(const float* qbar, const uint16_t* kc, int64_t npad, const float* kc_mean,
                  const float* kc_var, int64_t B, int64_t T, int64_t H, int64_t D,
                  int64_t block, float scale, float tau, int mode, int64_t sink_kv_lo,
                  int64_t sink_kv_hi, int64_t sink_q_lo, int64_t sink_q_hi, float* thr,
                  int32_t* counts, uint32_t* mask, solattn_stream_t stream);

/* ----------------------------------------------------------------- quant --
 * Per-token INT8 of a BTHD bf16 tensor, optionally smoothed by mean [B, H, D]:
 *   y = x - mean; s = max|y| / 127; s = s > 1e-8 ? s : 1e-8
 *   code = clamp(y/s >= 0 ? trunc(y/s + 0.5) : trunc(y/s - 0.5), -127, 127)
 * xi: int8 [B, TP, H, D]; xs: fp32 [B, TP, H]; rows t >= T are not written.
 * Replaces: _quant_kernel / quantize_bthd, /root/reference/_fused_quant.py:8-58
 * (and the Q half of _q_quant_threshold_kernel, _fused_prep.py:42-48). */
int solattn_quant_rows(const uint16_t* x, int64_t sx_b, int64_t sx_t, int64_t sx_h,
                       int64_t B, int64_t T, int64_t H, int64_t D, const float* mean,
                       int8_t* xi, float* xs, int64_t TP, solattn_stream_t stream);

/* Tokens per scale of the per-block INT8 variant below. */
#define SOLATTN_QUANT_BLOCK 128

/* solattn_quant_rows with one scale per block of SOLATTN_QUANT_BLOCK tokens
 * (per batch and head) instead of one per token: s = max(fl(amax / 127),
 * 1e-8) with amax the |max| of y over the block's tokens and channels, the
 * same code rule, and s written to xs for every token of the block. No
 * counterpart in the reference, which quantises Q and K per token: this is
 * BASELINE config 3's "Q/K quantised per 128-token block" wording, reported
 * beside the per-token parity mode. */
int solattn_quant_rows_blocked(const uint16_t* x, int64_t sx_b, int64_t sx_t, int64_t sx_h,
                               int64_t B, int64_t T, int64_t H, int64_t D, const float* mean,
                               int8_t* xi, float* xs, int64_t TP, solattn_stream_t stream);

/* Per-channel INT8 of V with vscale fp32 [B, H, D]:
 *   code = clamp(round_half_away(v / vscale[d]), -127, 127); vi: int8 [B, TP, H, D].
 * Replaces: _quant_v_kernel / quantize_v_per_channel,
 * /root/reference/_fused_quant.py:61-113. */
int solattn_quant_v(const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                    int64_t T, int64_t H, int64_t D, const float* vscale, int8_t* vi,
                    int64_t TP, solattn_stream_t stream);

/* ------------------------------------------------------- single-read INT8 --
 * The INT8 path's preparation with one read of q, k and v: pooled keys and
 * values, query centroids, centred kc and its moments (solattn_moments with
 * centre = 1), the V scale, per-token Q codes, per-token K codes smoothed by
 * kc_mean and (vscale != NULL) per-channel V codes -- the outputs of
 * solattn_pool + solattn_moments + solattn_quant_rows / solattn_quant_v, bit
 * for bit. Each head's K and V rows stay in registers until its moments are
 * known: the launch is cooperative (all workgroups resident) and the
 * workgroups of a head meet at two barriers in device memory. Returns
 * SOLATTN_EUNSUPPORTED when fewer than two heads' rows fit on the device at
 * once (or D != 128); the caller then uses the two-pass entry points.
 * vamax_part: fp32 [B, NT, H, D] scratch (with vscale); ks: [B, H, TP]
 * (ks_head_major != 0) or [B, TP, H]; sync: device scratch of at least
 * solattn_prep_int8_sync_bytes(B, H) bytes, reset by the call itself; its
 * first uint32 is nonzero after the call only if a barrier was not met within
 * ~0.1 s (results then invalid), which cannot happen with every workgroup
 * resident.
 * Replaces: fused_preprocess, /root/reference/_fused_prep.py:62-98, which reads
 * K and V twice. */
int64_t solattn_prep_int8_sync_bytes(int64_t B, int64_t H);
int solattn_prep_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                      const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                      const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h, int64_t B,
                      int64_t T, int64_t H, int64_t D, int64_t block, uint16_t* kc,
                      uint16_t* vc, int64_t npad, float* qbar, float* kc_mean, float* kc_var,
                      float* vamax_part, float* vscale, int8_t* qi, float* qs, int8_t* ki,
                      float* ks, int ks_head_major, int8_t* vi, int64_t TP, void* sync,
                      int64_t sync_bytes, solattn_stream_t stream);

/* ------------------------------------------------------------- forwards --
 * Sparse attention over exact blocks (flash attention on MFMA) plus the pooled
 * branch (one pooled key kc_j and value vc_j per approximate block, softmax
 * weight times len_j), one online softmax per query row.
 * counts/mask come from solattn_route for the same B, T, H and block. Each
 * workgroup builds its tile list from its mask row (mask bits at or past NT
 * are ignored, so any mask contents stay inside the tensors); counts only
 * order the dispatch (longest query blocks first). o: bf16, element
 * (b, t, h, d) at o + b*so_b + t*so_t + h*so_h + d, 16-byte aligned with
 * strides multiples of 8 elements (rows are written as 16-byte stores); rows
 * t >= T are not written.
 * Replaces: _forward_ptr + sol_attn, /root/reference/_tri_fwd.py:215-410. */
int solattn_fwd_bf16(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                     const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                     const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                     const uint16_t* kc, const uint16_t* vc, int64_t npad,
                     const int32_t* counts, const uint32_t* mask,
                     int64_t B, int64_t T, int64_t H, int64_t D, int64_t block, float scale,
                     uint16_t* o, int64_t so_b, int64_t so_t, int64_t so_h,
                     solattn_stream_t stream);

/* INT8 exact branch: S = int32(qi . ki) * (qs * c) * ks. int8_pv ==
 * SOLATTN_PV_BF16 runs P.V in bf16 against v, with P rounded to bf16 as in
 * solattn_fwd_bf16.
 * SOLATTN_PV_INT8 quantises P per row against the row max of each routed block:
 *   code = v_cvt_pk_u8_f32(exp2(s + log2(127) - rowmax_blk))
 * i.e. round to nearest, ties to even, of 127 * exp2(s - rowmax_blk) (at most
 * 127 by construction); the products int32(code . vi) are scaled by
 * (beta / 127) * vscale[d] with beta = exp2(rowmax_blk - m). The softmax
 * denominator adds the integer codes themselves, times beta / 127, so it is
 * the sum of the quantised P that the P.V multiplies.
 * Deliberate departures from /root/reference/_int8_fwd.py:348-353, which
 * rounds trunc(pe * 127 + 0.5) and sums the fp32 pe: the rounding rule and the
 * code-sum denominator (both within the INT8 tolerance, cosine >= 0.999), and,
 * at block 128, a ragged last block whose tiles take the max of each 64-key
 * tile instead of the whole block's.
 * SOLATTN_PV_INT8_RUNNING quantises P against the row's running max instead,
 * an integer m_int (log2 domain) at or above every scaled score seen:
 *   code = v_cvt_pk_u8_f32(exp2(s + log2(127) - m_int))
 * so the products of all exact blocks accumulate in int32 with no per-block
 * conversion; a block whose row max exceeds m_int raises it to ceil(max),
 * shifts the int32 sums right by the difference (floor) and scales the code
 * sum, kept in fp32, by the same power of two (exact); when a lane's half of
 * a row's code sum exceeds 2^23, m_int rises by one more, so the sums (at
 * most 127 times the code sum) stay below 2^31. After the exact blocks O = sums * vscale[d] / 127 and l = code sum /
 * 127, relative to 2^m_int. Codes of blocks below the
 * running max are coarser than against their own max: a further departure
 * from the reference, within the INT8 tolerance (cosine >= 0.999 per query
 * block against the reference arithmetic).
 * The pooled branch is BF16 as above (q, kc, vc); routing inputs as for
 * solattn_fwd_bf16. qi/ki/vi int8 [B, TP, H, D]; qs/ks fp32 [B, TP, H].
 * Replaces: _forward_int8_ptr + sol_attn_int8, /root/reference/_int8_fwd.py:208-432. */
int solattn_fwd_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                     const int8_t* qi, const float* qs, const int8_t* ki, const float* ks,
                     const int8_t* vi, const float* vscale, const uint16_t* v, int64_t sv_b,
                     int64_t sv_t, int64_t sv_h, int64_t TP, const uint16_t* kc,
                     const uint16_t* vc, int64_t npad, const int32_t* counts,
                     const uint32_t* mask, int64_t B, int64_t T,
                     int64_t H, int64_t D, int64_t block, float scale, int int8_pv,
                     uint16_t* o, int64_t so_b, int64_t so_t, int64_t so_h,
                     solattn_stream_t stream);

/* ------------------------------------------------------ whole pipeline --
 * sol_attn in one call: pool -> moments -> route -> fwd_bf16, with every
 * intermediate carved out of a caller-owned device workspace of at least
 * solattn_sol_attn_workspace_bytes(...) bytes (256-byte aligned base).
 * Replaces: sol_attn, /root/reference/_tri_fwd.py:354-410. */
int64_t solattn_sol_attn_workspace_bytes(int64_t B, int64_t T, int64_t H, int64_t D,
                                         int64_t block, int int8);
int solattn_sol_attn(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                     const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                     const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                     int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                     float scale, float tau, int64_t sink_kv_lo, int64_t sink_kv_hi,
                     int64_t sink_q_lo, int64_t sink_q_hi, void* workspace,
                     int64_t workspace_bytes, uint16_t* o, int64_t so_b, int64_t so_t,
                     int64_t so_h, solattn_stream_t stream);

/* sol_attn_int8 in one call: pool -> moments(centre) -> route(mode 1) ->
 * quant(q, k smoothed, v) -> fwd_int8. Replaces: sol_attn_int8,
 * /root/reference/_int8_fwd.py:379-432. */
int solattn_sol_attn_int8(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                          const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                          const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                          int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                          float scale, float tau, int64_t sink_kv_lo, int64_t sink_kv_hi,
                          int64_t sink_q_lo, int64_t sink_q_hi, int int8_pv,
                          void* workspace, int64_t workspace_bytes, uint16_t* o,
                          int64_t so_b, int64_t so_t, int64_t so_h,
                          solattn_stream_t stream);

/* solattn_sol_attn_int8 with Q and smoothed K quantised per
 * SOLATTN_QUANT_BLOCK-token block (solattn_quant_rows_blocked) instead of per
 * token; V, routing and the forward as there. No counterpart in the
 * reference: the config 3 variant above. */
int solattn_sol_attn_int8_qblock(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                                 const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                                 const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                                 int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                                 float scale, float tau, int64_t sink_kv_lo, int64_t sink_kv_hi,
                                 int64_t sink_q_lo, int64_t sink_q_hi, int int8_pv,
                                 void* workspace, int64_t workspace_bytes, uint16_t* o,
                                 int64_t so_b, int64_t so_t, int64_t so_h,
                                 solattn_stream_t stream);

/* ------------------------------------------------ allocation-free BF16 --
 * solattn_sol_attn without a workspace argument, for callers that cannot
 * allocate device memory (code under HIP graph capture, serving loops and
 * harnesses that forbid hipMalloc). No counterpart in the reference: it exists
 * for those callers only. The intermediates live in one fixed array of
 * SOLATTN_NOALLOC_SCRATCH_BYTES per device (held from the library's first use
 * on that device until the process ends); shapes whose intermediates exceed it
 * (solattn_sol_attn_workspace_bytes(B, T, H, D, block, 0) >
 * SOLATTN_NOALLOC_SCRATCH_BYTES) return SOLATTN_ESIZE. Every call on one
 * device shares that array: calls that overlap on one device (different
 * streams, or threads without ordering) race and must be serialised by the
 * caller. Nothing in the array needs clearing between calls. Same arguments,
 * results and errors as solattn_sol_attn otherwise; the device is the current
 * one. 32 MiB covers a B1 H40 T75600 call at block 128 (26 MiB) and a B1 H24
 * T32760 call at either block size (13 MiB at block 64). */
#define SOLATTN_NOALLOC_SCRATCH_BYTES (32ll << 20)
int solattn_sol_attn_noalloc(const uint16_t* q, int64_t sq_b, int64_t sq_t, int64_t sq_h,
                             const uint16_t* k, int64_t sk_b, int64_t sk_t, int64_t sk_h,
                             const uint16_t* v, int64_t sv_b, int64_t sv_t, int64_t sv_h,
                             int64_t B, int64_t T, int64_t H, int64_t D, int64_t block,
                             float scale, float tau, int64_t sink_kv_lo, int64_t sink_kv_hi,
                             int64_t sink_q_lo, int64_t sink_q_hi, uint16_t* o, int64_t so_b,
                             int64_t so_t, int64_t so_h, solattn_stream_t stream);

#ifdef __cplusplus
}
#endif
#endif /* SOLATTN_H */
