"""CPU oracle for the Sol-Attn sparse attention path -- TEST INFRASTRUCTURE.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this module, and only as the checker (or the timed CPU
baseline). The product path never imports it.

Two layers:

* ``liboracle.so`` (``oracle/solattn_oracle.c``): Morton permutation, pooling,
  moments, thresholds, routing and INT8 quantisation in the fixed operation
  order of ``include/solattn.h`` -- the HIP kernels must match these bit for
  bit.
* numpy / torch-fp32 restatements of the two forwards:
  ``forward_port`` / ``forward_int8_port`` follow the reference's loop
  (``/root/reference/_tri_fwd.py:268-345``, ``/root/reference/_int8_fwd.py:275-370``)
  group by group, including the bf16 rounding of P before P.V;
  ``forward_closed_form`` is the independent float64 pin: softmax over an
  augmented key set (tokens of exact blocks with bias 0, one pooled key
  ``kc_j`` per approximate block with value ``vc_j / len_j`` and bias
  ``ln(len_j)``).

Arrays in and out are numpy; bf16 tensors travel as ``uint16`` bit patterns.
"""

from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

__all__ = [
    "LOG2E", "lib", "f32_to_bf16", "bf16_to_f32", "morton_perm", "pool", "moments",
    "threshold", "route", "route_scores", "quant_rows", "quant_v", "prepare",
    "exact_matrix", "forward_port", "forward_int8_port", "forward_closed_form",
    "forward_dense_block_mask", "masked_attention_torch", "num_blocks", "npad_for",
    "routed_flops", "tie_count",
]

LOG2E = 1.4426950408889634
_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle.so")
_lib = None

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p


def lib() -> ctypes.CDLL:
    """Load (building with make if needed) the C oracle."""
    global _lib
    if _lib is None:
        if not os.path.exists(_SO):
            subprocess.run(["make", "-s", "-C", _HERE], check=True)
        L = ctypes.CDLL(_SO)
        L.or_morton_perm.argtypes = [_i64, _i64, _i64, ctypes.c_int, _i64, _vp, _vp]
        L.or_morton_perm.restype = ctypes.c_int
        L.or_pool.argtypes = [_vp, _i64, _i64, _i64] * 3 + [_i64] * 5 + [_vp, _vp, _i64, _vp, _vp]
        L.or_pool.restype = None
        L.or_moments.argtypes = [_vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_int, _vp, _vp, _vp, _vp]
        L.or_moments.restype = None
        L.or_threshold.argtypes = [_vp, _vp, _vp, _i64, _i64, _i64, _i64, ctypes.c_float,
                                   ctypes.c_float, ctypes.c_int, _vp]
        L.or_threshold.restype = None
        L.or_route.argtypes = [_vp, _vp, _i64, _vp, _i64, _i64, _i64, _i64, _i64, ctypes.c_float,
                               _i64, _i64, _i64, _i64, _vp, _vp, _vp, _vp]
        L.or_route.restype = None
        L.or_quant_rows.argtypes = [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _vp, _i64]
        L.or_quant_rows.restype = None
        L.or_quant_rows_blocked.argtypes = [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp,
                                            _vp, _vp, _i64, _i64]
        L.or_quant_rows_blocked.restype = None
        L.or_quant_v.argtypes = [_vp, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _vp, _vp, _i64]
        L.or_quant_v.restype = None
        L.or_f2bf.argtypes = [ctypes.c_float]
        L.or_f2bf.restype = ctypes.c_uint16
        _lib = L
    return _lib


def _p(a):
    return None if a is None else a.ctypes.data


def _estrides(a):
    """Element strides of a BTHD numpy array whose last dim is contiguous."""
    assert a.strides[-1] == a.itemsize, "last dim must be contiguous"
    return [s // a.itemsize for s in a.strides[:3]]


# --------------------------------------------------------------------- bf16
def f32_to_bf16(x) -> np.ndarray:
    """Round-to-nearest-even float32 -> bf16 bit patterns (uint16)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(h) -> np.ndarray:
    return (np.asarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def num_blocks(T: int, block: int) -> int:
    return (int(T) + block - 1) // block


def npad_for(NT: int) -> int:
    """kc/vc block padding: /root/reference/_preprocess.py:15,185."""
    return (NT + 63) // 64 * 64


# ------------------------------------------------------------------- Morton
def morton_perm(grid, curve: str = "3d", roll: int = 0):
    """(perm, inverse) int64; /root/reference/_morton.py:35-73 (+ roll,
    /root/reference/_morton_h3.py:50-53)."""
    f, h, w = (int(g) for g in grid)
    n = f * h * w
    perm = np.empty(n, np.int64)
    inv = np.empty(n, np.int64)
    rc = lib().or_morton_perm(f, h, w, 1 if curve == "2d_frame" else 0, int(roll), _p(perm), _p(inv))
    assert rc == 0
    return perm, inv


# --------------------------------------------------------------------- prep
def pool(q, k, v, block: int, npad: int | None = None, want_amax: bool = False):
    """kc, vc (bf16 bits [B,npad,H,D]), qbar (f32 [B,H,NT,D]), vamax_part."""
    B, T, H, D = q.shape
    NT = num_blocks(T, block)
    npad = npad_for(NT) if npad is None else npad
    kc = np.zeros((B, npad, H, D), np.uint16)
    vc = np.zeros((B, npad, H, D), np.uint16)
    qbar = np.zeros((B, H, NT, D), np.float32)
    amax = np.zeros((B, NT, H, D), np.float32) if want_amax else None
    lib().or_pool(_p(q), *_estrides(q), _p(k), *_estrides(k), _p(v), *_estrides(v),
                  B, T, H, D, block, _p(kc), _p(vc), npad, _p(qbar), _p(amax))
    return kc, vc, qbar, amax


def moments(kc, NT: int, centre: bool, vamax_part=None):
    """Returns (kc (a centred copy when centre), mean, var, vscale)."""
    kc = np.ascontiguousarray(kc).copy()
    B, npad, H, D = kc.shape
    mean = np.zeros((B, H, D), np.float32)
    var = np.zeros((B, H, D), np.float32)
    vscale = np.zeros((B, H, D), np.float32) if vamax_part is not None else None
    lib().or_moments(_p(kc), npad, B, NT, H, D, int(bool(centre)), _p(mean), _p(var),
                     _p(vamax_part), _p(vscale))
    return kc, mean, var, vscale


def threshold(qbar, mean, var, scale: float, tau: float, mode: int):
    B, H, NT, D = qbar.shape
    thr = np.zeros((B, NT, H), np.float32)
    lib().or_threshold(_p(qbar), _p(mean), _p(var), B, NT, H, D, float(scale), float(tau),
                       int(mode), _p(thr))
    return thr


def route(qbar, kc, thr, T: int, block: int, scale: float, sink_kv=(0, 0), sink_q=(0, 0),
          want_scores: bool = False):
    """counts int32 [B,H,NT], lists int16 [B,H,NT,NT], mask uint32 [B,H,NT,W]."""
    B, H, NT, D = qbar.shape
    npad = kc.shape[1]
    W = (NT + 31) // 32
    counts = np.zeros((B, H, NT), np.int32)
    lists = np.zeros((B, H, NT, NT), np.int16)
    mask = np.zeros((B, H, NT, W), np.uint32)
    scores = np.zeros((B, H, NT, NT), np.float32) if want_scores else None
    lib().or_route(_p(qbar), _p(np.ascontiguousarray(kc)), npad, _p(thr), B, T, H, D, block,
                   float(scale), int(sink_kv[0]), int(sink_kv[1]), int(sink_q[0]), int(sink_q[1]),
                   _p(counts), _p(lists), _p(mask), _p(scores))
    return counts, lists, mask, scores


def route_scores(qbar, kc, scale):
    """float64 closed form of R[i][j] = c * (qbar_i . kc_j) -- an independent pin."""
    c = float(np.float32(scale) * np.float32(LOG2E))
    kcf = bf16_to_f32(kc).astype(np.float64)
    NT = qbar.shape[2]
    return np.einsum("bhid,bjhd->bhij", qbar.astype(np.float64), kcf[:, :NT]) * c


def tie_count(scores, thr, exact_a, exact_b, ulps: int = 8):
    """Pairs that differ between two exact-matrices and whether every such pair
    lies inside the tie band |R - thr| <= ulps * ulp(max(|R|, |thr|))."""
    B, H, NT, _ = scores.shape
    t = np.transpose(thr, (0, 2, 1))[..., None]  # [B,H,NT,1]
    mag = np.maximum(np.abs(scores), np.abs(t)).astype(np.float32)
    band = np.abs(scores - t) <= ulps * np.spacing(mag)
    diff = exact_a != exact_b
    return int(diff.sum()), bool(np.all(band[diff]))


def quant_rows(x, mean=None, TP: int | None = None, block: int | None = None):
    """Per-token codes and scales (the reference's), or with ``block`` one scale
    per block of that many tokens (BASELINE config 3's variant), written for
    every token of the block."""
    B, T, H, D = x.shape
    TP = T if TP is None else TP
    xi = np.zeros((B, TP, H, D), np.int8)
    xs = np.zeros((B, TP, H), np.float32)
    if block is None:
        lib().or_quant_rows(_p(x), *_estrides(x), B, T, H, D, _p(mean), _p(xi), _p(xs), TP)
    else:
        lib().or_quant_rows_blocked(_p(x), *_estrides(x), B, T, H, D, _p(mean), _p(xi), _p(xs),
                                    TP, int(block))
    return xi, xs


def quant_v(v, vscale, TP: int | None = None):
    B, T, H, D = v.shape
    TP = T if TP is None else TP
    vi = np.zeros((B, TP, H, D), np.int8)
    lib().or_quant_v(_p(v), *_estrides(v), B, T, H, D, _p(vscale), _p(vi), TP)
    return vi


def prepare(q, k, v, *, block: int, scale: float | None = None, tau: float = 1.0,
            int8: bool = False, sink_kv=(0, 0), sink_q=(0, 0), int8_pv: bool = True,
            want_scores: bool = False, quant_block: int | None = None):
    """The whole pre-forward pipeline: BF16 ``prepare`` (/root/reference/_preprocess.py:268)
    or INT8 ``fused_preprocess`` (/root/reference/_fused_prep.py:62)."""
    B, T, H, D = q.shape
    scale = D ** -0.5 if scale is None else float(scale)
    NT = num_blocks(T, block)
    kc, vc, qbar, amax = pool(q, k, v, block, want_amax=int8 and int8_pv)
    kc, mean, var, vscale = moments(kc, NT, centre=int8, vamax_part=amax)
    thr = threshold(qbar, mean, var, scale, tau, 1 if int8 else 0)
    counts, lists, mask, scores = route(qbar, kc, thr, T, block, scale, sink_kv, sink_q,
                                        want_scores)
    out = dict(block=block, scale=scale, tau=tau, T=T, NT=NT, kc=kc, vc=vc, qbar=qbar,
               kc_mean=mean, kc_var=var, thr=thr, counts=counts, lists=lists, mask=mask,
               scores=scores, vamax_part=amax, int8=int8)
    if int8:
        qi, qs = quant_rows(q, block=quant_block)
        ki, ks = quant_rows(k, mean=mean, block=quant_block)
        out.update(qi=qi, qs=qs, ki=ki, ks=ks)
        if int8_pv:
            out.update(vi=quant_v(v, vscale), vscale=vscale)
    return out


def exact_matrix(mask, NT: int) -> np.ndarray:
    """bool [B,H,NT,NT] from the packed bitmask."""
    j = np.arange(NT)
    words = mask[..., j >> 5]
    return ((words >> (j & 31).astype(np.uint32)) & 1).astype(bool)


# ------------------------------------------------------------------ forward
def _rows(T, block, i):
    lo = i * block
    return lo, min(block, T - lo)


def _bf16_round(x):
    return bf16_to_f32(f32_to_bf16(x))


def forward_port(q, k, v, prep, rows, group: int = 64, round_p: bool = True):
    """The reference's BF16 forward loop for the query blocks ``rows``
    [(b, h, i), ...]; /root/reference/_tri_fwd.py:248-347. Returns
    {(b,h,i): float32 [len_i, D]}. ``round_p=False`` skips the bf16 rounding of
    P (used to pin the algebra against the closed form)."""
    block, T, NT = prep["block"], prep["T"], prep["NT"]
    c = np.float32(np.float32(prep["scale"]) * np.float32(LOG2E))
    ex = exact_matrix(prep["mask"], NT)
    tail = np.float32(T - (NT - 1) * block)
    rnd = _bf16_round if round_p else (lambda a: a)
    out = {}
    for (b, h, i) in rows:
        lo, ln = _rows(T, block, i)
        qb = np.zeros((block, q.shape[3]), np.float32)
        qb[:ln] = bf16_to_f32(q[b, lo:lo + ln, h])
        m = np.full(block, -np.inf, np.float32)
        l = np.zeros(block, np.float32)
        acc = np.zeros((block, q.shape[3]), np.float32)
        for g0 in range(0, NT, group):
            idx = g0 + np.arange(group)
            valid = idx < NT
            sel = np.minimum(idx, prep["kc"].shape[1] - 1)
            kcg = bf16_to_f32(prep["kc"][b, sel, h])
            vcg = bf16_to_f32(prep["vc"][b, sel, h])
            scores = (qb @ kcg.T).astype(np.float32) * c
            exact = np.zeros(group, bool)
            exact[valid] = ex[b, h, i, idx[valid]]
            approx = valid & ~exact
            asc = np.where(approx[None, :], scores, -np.inf).astype(np.float32)
            new_max = np.maximum(m, asc.max(axis=1))
            with np.errstate(invalid="ignore"):
                alpha = np.exp2(np.where(m == new_max, np.float32(0), m - new_max)).astype(np.float32)
                p = np.where(approx[None, :], np.exp2(asc - new_max[:, None]), 0).astype(np.float32)
            acc = acc * alpha[:, None] + rnd(p) @ vcg
            lengths = np.where(idx == NT - 1, tail, np.float32(block)).astype(np.float32)
            l = l * alpha + (p * lengths[None, :]).sum(axis=1, dtype=np.float32)
            m = new_max
            for off in np.nonzero(exact)[0]:
                j = g0 + int(off)
                klo, kln = _rows(T, block, j)
                kb = np.zeros((block, q.shape[3]), np.float32)
                vb = np.zeros((block, q.shape[3]), np.float32)
                kb[:kln] = bf16_to_f32(k[b, klo:klo + kln, h])
                vb[:kln] = bf16_to_f32(v[b, klo:klo + kln, h])
                s = (qb @ kb.T).astype(np.float32) * c
                s[:, kln:] = -np.inf
                new_max = np.maximum(m, s.max(axis=1))
                alpha = np.exp2(m - new_max).astype(np.float32)
                p = np.exp2(s - new_max[:, None]).astype(np.float32)
                l = l * alpha + p.sum(axis=1, dtype=np.float32)
                acc = acc * alpha[:, None] + rnd(p) @ vb
                m = new_max
        out[(b, h, i)] = (acc / l[:, None])[:ln].astype(np.float32)
    return out


def forward_int8_port(q, v, prep, rows, int8_pv: bool = True, group: int = 64,
                      codes: str = "reference"):
    """The reference's INT8 forward loop, /root/reference/_int8_fwd.py:242-372:
    BF16 routing and pooled branch on centred kc; exact branch from qi/qs, ki/ks
    (int32 dot), P.V in int8 against the block max (int8_pv) or in bf16.

    ``codes`` selects the int8 P.V arithmetic:
      "reference": pi = trunc(min(pe*127 + 0.5, 127)), row sum += beta * sum(pe)
                   (/root/reference/_int8_fwd.py:348-353);
      "kernel":    pi = round-half-even(exp2(s + log2(127) - bm)), row sum +=
                   beta/127 * sum(pi), and at block 128 a ragged last block of
                   more than 64 keys quantised per 64-key tile, each against its
                   own max -- the HIP kernel's documented departure (the softmax
                   denominator is that of the quantised P the P.V multiplies);
      "running":   the HIP kernel's SOLATTN_PV_INT8_RUNNING arithmetic
                   (``_forward_int8_running``), int8_pv only."""
    assert codes in ("reference", "kernel", "running")
    if codes == "running":
        assert int8_pv, "running codes are an int8 P.V arithmetic"
        return _forward_int8_running(q, v, prep, rows)
    block, T, NT = prep["block"], prep["T"], prep["NT"]
    D = q.shape[3]
    c = np.float32(np.float32(prep["scale"]) * np.float32(LOG2E))
    ex = exact_matrix(prep["mask"], NT)
    tail = np.float32(T - (NT - 1) * block)
    inv127 = np.float32(1.0 / 127.0)
    out = {}
    for (b, h, i) in rows:
        lo, ln = _rows(T, block, i)
        qb = np.zeros((block, D), np.float32)
        qb[:ln] = bf16_to_f32(q[b, lo:lo + ln, h])
        qi = np.zeros((block, D), np.int64)
        qi[:ln] = prep["qi"][b, lo:lo + ln, h]
        qs = np.zeros(block, np.float32)
        qs[:ln] = prep["qs"][b, lo:lo + ln, h]
        qs_log2 = (qs * c).astype(np.float32)
        if int8_pv:
            vsc = prep["vscale"][b, h].astype(np.float32)
        m = np.full(block, -np.inf, np.float32)
        l = np.zeros(block, np.float32)
        acc = np.zeros((block, D), np.float32)
        for g0 in range(0, NT, group):
            idx = g0 + np.arange(group)
            valid = idx < NT
            sel = np.minimum(idx, prep["kc"].shape[1] - 1)
            kcg = bf16_to_f32(prep["kc"][b, sel, h])
            vcg = bf16_to_f32(prep["vc"][b, sel, h])
            scores = (qb @ kcg.T).astype(np.float32) * c
            exact = np.zeros(group, bool)
            exact[valid] = ex[b, h, i, idx[valid]]
            approx = valid & ~exact
            asc = np.where(approx[None, :], scores, -np.inf).astype(np.float32)
            new_max = np.maximum(m, asc.max(axis=1))
            with np.errstate(invalid="ignore"):
                alpha = np.exp2(np.where(m == new_max, np.float32(0), m - new_max)).astype(np.float32)
                p = np.where(approx[None, :], np.exp2(asc - new_max[:, None]), 0).astype(np.float32)
            acc = acc * alpha[:, None] + _bf16_round(p) @ vcg
            lengths = np.where(idx == NT - 1, tail, np.float32(block)).astype(np.float32)
            l = l * alpha + (p * lengths[None, :]).sum(axis=1, dtype=np.float32)
            m = new_max
            for off in np.nonzero(exact)[0]:
                j = g0 + int(off)
                klo, kln = _rows(T, block, j)
                # key ranges quantised against one max: the block, or (kernel
                # arithmetic, block 128) each 64-key tile of a ragged last block
                split = (codes == "kernel" and int8_pv and block == 128 and j == NT - 1
                         and 64 < kln < block)
                for slo, sln in ((0, 64), (64, kln - 64)) if split else ((0, kln),):
                    ki = np.zeros((block, D), np.int64)
                    ki[:sln] = prep["ki"][b, klo + slo:klo + slo + sln, h]
                    ks = np.zeros(block, np.float32)
                    ks[:sln] = prep["ks"][b, klo + slo:klo + slo + sln, h]
                    a32 = (qi @ ki.T).astype(np.float32)
                    s = (a32 * (qs_log2[:, None] * ks[None, :])).astype(np.float32)
                    s[:, sln:] = -np.inf
                    bm = s.max(axis=1)
                    new_max = np.maximum(m, bm)
                    alpha = np.exp2(m - new_max).astype(np.float32)
                    if int8_pv:
                        vi = np.zeros((block, D), np.int64)
                        vi[:sln] = prep["vi"][b, klo + slo:klo + slo + sln, h]
                        beta = np.exp2(bm - new_max).astype(np.float32)
                        if codes == "kernel":
                            x127 = np.exp2(s + np.float32(np.log2(127.0)) - bm[:, None]).astype(np.float32)
                            pi = np.clip(np.rint(x127), 0, 255).astype(np.int64)
                            l = l * alpha + (beta * inv127) * pi.sum(axis=1).astype(np.float32)
                        else:
                            pe = np.exp2(s - bm[:, None]).astype(np.float32)
                            l = l * alpha + beta * pe.sum(axis=1, dtype=np.float32)
                            pi = np.minimum(pe * np.float32(127) + np.float32(0.5),
                                            np.float32(127)).astype(np.int64)
                        pv = (pi @ vi).astype(np.float32) * ((beta * inv127)[:, None] * vsc[None, :])
                    else:
                        vb = np.zeros((block, D), np.float32)
                        vb[:sln] = bf16_to_f32(v[b, klo + slo:klo + slo + sln, h])
                        p = np.exp2(s - new_max[:, None]).astype(np.float32)
                        l = l * alpha + p.sum(axis=1, dtype=np.float32)
                        pv = _bf16_round(p) @ vb
                    acc = acc * alpha[:, None] + pv
                    m = new_max
        out[(b, h, i)] = (acc / l[:, None])[:ln].astype(np.float32)
    return out


RUN_LANE_SUM_LIMIT = 2.0 ** 23  # a lane's half of the code sum before the max rises


def _forward_int8_running(q, v, prep, rows):
    """INT8 forward with P codes against the row's running max
    (SOLATTN_PV_INT8_RUNNING; a departure from /root/reference/_int8_fwd.py:
    333-353, which quantises against each block's max). In the HIP kernels'
    unit order -- block 128: the full exact blocks ascending, then the tiles
    of a ragged last block (64 keys each); block 64: the ragged last tile
    first, then the full tiles ascending -- each unit u:
      m' = max(m, ceil(max_row s_u)), +1 when either half of the row's code
      sum (keys k with k mod 8 < 4, the rest: the two lanes of a row) exceeds
      2^23 (the int32 sums' headroom),
      sums >>= (m' - m) (arithmetic shift, floor), code sums *= 2^-(m' - m)
      (exact: the kernels keep them in fp32),
      pi = round-half-even(exp2(s_u + log2(127) - m')) (at most 127),
      sums += pi . vi (int32), code sum += sum(pi);
    in the kernels' fp32 operation order: s_u = fl(int32 * ks) * qsl with qsl =
    fl(qs * c), the row max fl(max(fl(int32 * ks)) * qsl), and the exponent
    one fma(fl(int32 * ks), qsl, fl(log2(127) - m')), so that P codes flip
    between the two only where exp2's own rounding lands on a half;
    then O = sums * vscale / 127, l = code sum / 127 relative to 2^m, and the
    pooled tiles (64-block chunks) in fp32 as the BF16 forward."""
    block, T, NT = prep["block"], prep["T"], prep["NT"]
    D = q.shape[3]
    c = np.float32(np.float32(prep["scale"]) * np.float32(LOG2E))
    ex = exact_matrix(prep["mask"], NT)
    tail = np.float32(T - (NT - 1) * block)
    inv127 = np.float32(1.0 / 127.0)
    log2_127 = np.float32(np.log2(127.0))
    ragged = T % block != 0
    out = {}
    for (b, h, i) in rows:
        lo, ln = _rows(T, block, i)
        qb = np.zeros((block, D), np.float32)
        qb[:ln] = bf16_to_f32(q[b, lo:lo + ln, h])
        qi = np.zeros((block, D), np.int64)
        qi[:ln] = prep["qi"][b, lo:lo + ln, h]
        qs = np.zeros(block, np.float32)
        qs[:ln] = prep["qs"][b, lo:lo + ln, h]
        qsl = (qs * c).astype(np.float32)
        vsc = prep["vscale"][b, h].astype(np.float32)
        exact = [int(j) for j in np.nonzero(ex[b, h, i])[0]]
        units = []  # (first key, keys)
        full = [j for j in exact if not (ragged and j == NT - 1)]
        rag = [j for j in exact if ragged and j == NT - 1]
        if block == 128:
            units = [(j * block, block) for j in full]
            for j in rag:
                kln = T - j * block
                units += [(j * block + o, min(64, kln - o)) for o in range(0, kln, 64)]
        else:
            units = [(j * block, T - j * block) for j in rag] + [(j * block, block) for j in full]
        m = np.full(block, -np.inf, np.float32)
        acc = np.zeros((block, D), np.int64)
        lsum = np.zeros((block, 2), np.float64)  # per lane half
        for k0, kn in units:
            ki = np.zeros((kn, D), np.int64)
            ki[:] = prep["ki"][b, k0:k0 + kn, h]
            ks = prep["ks"][b, k0:k0 + kn, h].astype(np.float32)
            sk = ((qi @ ki.T).astype(np.float32) * ks[None, :]).astype(np.float32)
            bmax = (sk.max(axis=1) * qsl).astype(np.float32)
            m_new = np.maximum(m, np.ceil(bmax)).astype(np.float32)
            m_new = m_new + (lsum.max(axis=1) > RUN_LANE_SUM_LIMIT).astype(np.float32)
            with np.errstate(invalid="ignore"):
                d = np.where(np.isinf(m), 31, np.minimum(m_new - m, 31)).astype(np.int64)
            acc >>= d[:, None]
            lsum = np.ldexp(lsum, -d[:, None])
            m = m_new
            arg = (sk.astype(np.float64) * qsl[:, None].astype(np.float64)
                   + (log2_127 - m).astype(np.float64)[:, None]).astype(np.float32)  # one fma
            x127 = np.exp2(arg.astype(np.float64)).astype(np.float32)
            pi = np.rint(x127).astype(np.int64)
            assert pi.max() <= 127
            vi = prep["vi"][b, k0:k0 + kn, h].astype(np.int64)
            acc += pi @ vi
            upper = (np.arange(kn) % 8) >= 4
            lsum[:, 0] += pi[:, ~upper].sum(axis=1)
            lsum[:, 1] += pi[:, upper].sum(axis=1)
            assert np.abs(acc).max() < 2 ** 31
        accf = (acc.astype(np.float32) * (vsc * inv127)[None, :]).astype(np.float32)
        l = (lsum.sum(axis=1).astype(np.float32) * inv127).astype(np.float32)  # fp32 in the kernels
        for g0 in range(0, NT, 64):
            idx = np.arange(g0, min(g0 + 64, NT))
            approx = ~ex[b, h, i, idx]
            if not approx.any():
                continue
            idx = idx[approx]
            kcg = bf16_to_f32(prep["kc"][b, idx, h])
            vcg = bf16_to_f32(prep["vc"][b, idx, h])
            sc = ((qb @ kcg.T).astype(np.float32) * c).astype(np.float32)
            nm = np.maximum(m, sc.max(axis=1))
            with np.errstate(invalid="ignore"):
                alpha = np.exp2(np.where(m == nm, np.float32(0), m - nm)).astype(np.float32)
            p = np.exp2(sc - nm[:, None]).astype(np.float32)
            lengths = np.where(idx == NT - 1, tail, np.float32(block)).astype(np.float32)
            accf = accf * alpha[:, None] + _bf16_round(p) @ vcg
            l = l * alpha + (p * lengths[None, :]).sum(axis=1, dtype=np.float32)
            m = nm
        out[(b, h, i)] = (accf / l[:, None])[:ln].astype(np.float32)
    return out


def forward_closed_form(q, k, v, prep, rows, qk=None):
    """float64 softmax over the augmented key set; an independent pin of the
    forward. ``qk`` optionally supplies dequantised (q, k) float arrays for the
    INT8 path's exact branch."""
    block, T, NT = prep["block"], prep["T"], prep["NT"]
    scale = float(np.float32(prep["scale"]))
    ex = exact_matrix(prep["mask"], NT)
    lens = np.array([min(block, T - j * block) for j in range(NT)], np.float64)
    out = {}
    for (b, h, i) in rows:
        lo, ln = _rows(T, block, i)
        qf = bf16_to_f32(q[b, lo:lo + ln, h]).astype(np.float64)
        if qk is not None:
            qx = qk[0][b, lo:lo + ln, h].astype(np.float64)
        exact = ex[b, h, i]
        tok = np.concatenate([np.arange(j * block, j * block + lens[j], dtype=np.int64)
                              for j in np.nonzero(exact)[0]]) if exact.any() else np.zeros(0, np.int64)
        kt = bf16_to_f32(k[b, tok, h]).astype(np.float64)
        vt = bf16_to_f32(v[b, tok, h]).astype(np.float64)
        ap = np.nonzero(~exact)[0]
        kcp = bf16_to_f32(prep["kc"][b, ap, h]).astype(np.float64)
        vcp = bf16_to_f32(prep["vc"][b, ap, h]).astype(np.float64) / lens[ap, None]
        if qk is not None:
            s_tok = (qx @ qk[1][b, tok, h].astype(np.float64).T) * scale
        else:
            s_tok = (qf @ kt.T) * scale
        s_pool = (qf @ kcp.T) * scale + np.log(lens[ap])[None, :]
        s = np.concatenate([s_tok, s_pool], axis=1)
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        o = (p @ np.concatenate([vt, vcp], axis=0)) / p.sum(axis=1, keepdims=True)
        out[(b, h, i)] = o
    return out


def forward_dense_block_mask(q, k, v, prep, rows):
    """Diagnostic only: dense softmax restricted to the exact blocks (the pooled
    term dropped). Not the reference's output."""
    block, T, NT = prep["block"], prep["T"], prep["NT"]
    scale = float(np.float32(prep["scale"]))
    ex = exact_matrix(prep["mask"], NT)
    out = {}
    for (b, h, i) in rows:
        lo, ln = _rows(T, block, i)
        qf = bf16_to_f32(q[b, lo:lo + ln, h]).astype(np.float64)
        tok = np.concatenate([np.arange(j * block, min(T, j * block + block))
                              for j in np.nonzero(ex[b, h, i])[0]])
        s = (qf @ bf16_to_f32(k[b, tok, h]).astype(np.float64).T) * scale
        s -= s.max(axis=1, keepdims=True)
        p = np.exp(s)
        out[(b, h, i)] = (p @ bf16_to_f32(v[b, tok, h]).astype(np.float64)) / p.sum(1, keepdims=True)
    return out


def masked_attention_torch(q, k, v, prep, heads=None, qblocks=None, threads=None):
    """The masked-attention CPU path in torch fp32, evaluated block-wise over
    query blocks (memory O(block * N)): SDPA over [tokens ; pooled keys] with an
    additive bias of 0 / ln(len_j) / -inf. Inputs are float32 torch tensors
    [B, T, H, D]; returns {(b,h,i): tensor [len_i, D]}."""
    import torch

    if threads:
        torch.set_num_threads(int(threads))
    block, T, NT = prep["block"], prep["T"], prep["NT"]
    B, _, H, D = q.shape
    scale = float(np.float32(prep["scale"]))
    ex = torch.from_numpy(exact_matrix(prep["mask"], NT))
    kc = torch.from_numpy(bf16_to_f32(prep["kc"][:, :NT]))
    vc = torch.from_numpy(bf16_to_f32(prep["vc"][:, :NT]))
    lens = torch.tensor([min(block, T - j * block) for j in range(NT)], dtype=torch.float32)
    tok_block = torch.arange(T) // block
    heads = range(H) if heads is None else heads
    qblocks = range(NT) if qblocks is None else qblocks
    out = {}
    neg = torch.tensor(float("-inf"))
    for b in range(B):
        for h in heads:
            keys = torch.cat([k[b, :, h], kc[b, :, h]], 0)
            vals = torch.cat([v[b, :, h], vc[b, :, h] / lens[:, None]], 0)
            for i in qblocks:
                lo, ln = _rows(T, block, i)
                e = ex[b, h, i]
                bias_tok = torch.where(e[tok_block], torch.tensor(0.0), neg)
                bias_pool = torch.where(e, neg, torch.log(lens))
                bias = torch.cat([bias_tok, bias_pool])[None, :]
                s = (q[b, lo:lo + ln, h] @ keys.T) * scale + bias
                out[(b, h, i)] = torch.softmax(s, dim=-1) @ vals
    return out


def routed_flops(counts_or_mask, T: int, block: int, D: int, mask: bool = False,
                 lists=None) -> float:
    """Algorithmic FLOPs of one forward on valid tokens:
    4*D*sum_{b,h,i} len_i * (sum_{j exact} len_j + |approx(i)|)."""
    NT = num_blocks(T, block)
    lens = np.array([min(block, T - j * block) for j in range(NT)], np.float64)
    ex = exact_matrix(counts_or_mask, NT) if mask else counts_or_mask
    exact_tok = (ex * lens[None, None, None, :]).sum(-1)
    n_approx = (~ex).sum(-1)
    return float(4 * D * (lens[None, None, :] * (exact_tok + n_approx)).sum())
