"""Fused preprocess for the INT8 path (host side).

Mirrors /root/reference/_fused_prep.py:62-98: pooled keys centred by their own
mean (K smoothing), thresholds tau*sigma, per-token INT8 Q and smoothed K,
per-channel INT8 V, all from the gfx950 kernels: two passes (pooling with the
Q codes, moments, then the K and V codes), or optionally one read of Q, K and
V (``solattn_prep_int8``, same bits, slower on this part).
"""

from __future__ import annotations

import torch

from ._capi import LIB, QUANT_BLOCK, SolAttnError, call, ptr, stream
from ._preprocess import (BLOCK_SIZE, GROUP_PAD, HEAD_DIM, Routing, as_kernel_input, check_inputs,
                          num_blocks, pad_heads, route)

SOLATTN_EUNSUPPORTED = -2

__all__ = ["fused_preprocess", "fused_preprocess_routing"]


def fused_preprocess_routing(q, k, v, *, tau, scale, int8_pv=True, block=BLOCK_SIZE,
                             sink_blocks=(0, 0), sink_q=(0, 0), quant_block=None,
                             single_read=False):
    """(Routing, qi, qs, ki, ks, vi) -- the INT8 path's inputs to the forward.
    Head dims below 128 run zero-padded; codes come back for the first D
    channels (the padded ones are 0). ``quant_block=128``: Q and K scales per
    128-token block (written for every token), as ``sol_attn_int8``.
    ``single_read=True`` prepares with one read of q, k and v
    (``solattn_prep_int8``; same bits) where the shape fits that schedule. It
    is off by default: on MI355X the two passes are faster at every measured
    shape."""
    if quant_block not in (None, QUANT_BLOCK):
        raise ValueError(f"quant_block must be None or {QUANT_BLOCK}, got {quant_block}")
    D0 = q.shape[-1]
    if D0 != HEAD_DIM:
        r, qi, qs, ki, ks, vi = fused_preprocess_routing(
            pad_heads(q), pad_heads(k), pad_heads(v), tau=tau, scale=scale, int8_pv=int8_pv,
            block=block, sink_blocks=sink_blocks, sink_q=sink_q, quant_block=quant_block)
        cut = lambda t: None if t is None else t[..., :D0]  # noqa: E731
        r = r._replace(kc=cut(r.kc), vc=cut(r.vc), qbar=cut(r.qbar), kc_mean=cut(r.kc_mean),
                       kc_var=cut(r.kc_var), vamax_part=cut(r.vamax_part), vscale=cut(r.vscale))
        return r, cut(qi), qs, cut(ki), ks, cut(vi)
    if single_read and quant_block is None:
        one = _single_read(q, k, v, tau=tau, scale=scale, int8_pv=int8_pv, block=block,
                           sink_blocks=sink_blocks, sink_q=sink_q)
        if one is not None:
            return one
    r: Routing = route(q, k, v, scale=scale, tau=tau, block=block, int8=True, v_absmax=int8_pv,
                       sink_blocks=sink_blocks, sink_q=sink_q)
    q, k, v = as_kernel_input(q), as_kernel_input(k), as_kernel_input(v)
    B, T, H, D = q.shape
    dev = q.device
    qi = torch.empty((B, T, H, D), device=dev, dtype=torch.int8)
    ki = torch.empty_like(qi)
    qs = torch.empty((B, T, H), device=dev, dtype=torch.float32)
    ks = torch.empty_like(qs)
    vi = torch.empty_like(qi) if int8_pv else None
    with torch.cuda.device(dev):
        s = stream(dev)
        rows = "solattn_quant_rows" if quant_block is None else "solattn_quant_rows_blocked"
        call(rows, ptr(q), q.stride(0), q.stride(1), q.stride(2), B, T, H, D, None, ptr(qi),
             ptr(qs), T, s)
        call(rows, ptr(k), k.stride(0), k.stride(1), k.stride(2), B, T, H, D, ptr(r.kc_mean),
             ptr(ki), ptr(ks), T, s)
        if int8_pv:
            call("solattn_quant_v", ptr(v), v.stride(0), v.stride(1), v.stride(2), B, T, H, D,
                 ptr(r.vscale), ptr(vi), T, s)
    return r, qi, qs, ki, ks, vi


def _single_read(q, k, v, *, tau, scale, int8_pv, block, sink_blocks, sink_q):
    """The outputs of fused_preprocess_routing from one read of q, k and v
    (``solattn_prep_int8``, then routing), or None when the shape does not fit
    the single-read schedule on this device (the caller runs the two passes)."""
    check_inputs(q, k, v, block, padded_ok=False)
    q, k, v = as_kernel_input(q), as_kernel_input(k), as_kernel_input(v)
    B, T, H, D = q.shape
    NT = num_blocks(T, block)
    npad = (NT + GROUP_PAD - 1) // GROUP_PAD * GROUP_PAD
    W = (NT + 31) // 32
    dev = q.device
    f32 = dict(device=dev, dtype=torch.float32)
    kc = torch.zeros((B, npad, H, D), device=dev, dtype=torch.bfloat16)
    vc = torch.zeros_like(kc)
    qbar = torch.empty((B, H, NT, D), **f32)
    kc_mean = torch.empty((B, H, D), **f32)
    kc_var = torch.empty((B, H, D), **f32)
    vamax = torch.empty((B, NT, H, D), **f32) if int8_pv else None
    vscale = torch.empty((B, H, D), **f32) if int8_pv else None
    qi = torch.empty((B, T, H, D), device=dev, dtype=torch.int8)
    ki = torch.empty_like(qi)
    vi = torch.empty_like(qi) if int8_pv else None
    qs = torch.empty((B, T, H), **f32)
    ks = torch.empty_like(qs)
    sync = torch.empty(LIB.solattn_prep_int8_sync_bytes(B, H), device=dev, dtype=torch.uint8)
    with torch.cuda.device(dev):
        s = stream(dev)
        rc = LIB.solattn_prep_int8(
            ptr(q), q.stride(0), q.stride(1), q.stride(2), ptr(k), k.stride(0), k.stride(1),
            k.stride(2), ptr(v), v.stride(0), v.stride(1), v.stride(2), B, T, H, D, block, ptr(kc),
            ptr(vc), npad, ptr(qbar), ptr(kc_mean), ptr(kc_var), ptr(vamax), ptr(vscale), ptr(qi),
            ptr(qs), ptr(ki), ptr(ks), 0, ptr(vi), T, ptr(sync), sync.numel(), s)
        if rc == SOLATTN_EUNSUPPORTED:
            return None
        if rc != 0:
            raise SolAttnError(f"solattn_prep_int8 failed ({rc}): "
                               f"{LIB.solattn_last_error().decode(errors='replace')}")
        thr = torch.empty((B, NT, H), **f32)
        counts = torch.empty((B, H, NT), device=dev, dtype=torch.int32)
        mask = torch.empty((B, H, NT, W), device=dev, dtype=torch.int32)
        call("solattn_route", ptr(qbar), ptr(kc), npad, None, ptr(kc_var), B, T, H, D, block,
             float(scale), float(tau), 1, int(sink_blocks[0]), int(sink_blocks[1]),
             int(sink_q[0]), int(sink_q[1]), ptr(thr), ptr(counts), ptr(mask), s)
    r = Routing(kc, vc, thr, qbar, kc_mean, kc_var, counts, mask, vamax, vscale, block, T)
    return r, qi, qs, ki, ks, vi


def fused_preprocess(q, k, v, *, tau, scale, tokens=None, int8_pv=True, block=BLOCK_SIZE):
    """Returns (kc, vc, threshold, qi, qs, ki, ks, vi, vsc) with K smoothed, as
    /root/reference/_fused_prep.py:62-98 (vsc is [B*H, D]; vi/vsc are None
    without int8_pv)."""
    if tokens is not None and tokens != q.shape[1]:
        q, k, v = q[:, :tokens], k[:, :tokens], v[:, :tokens]
    r, qi, qs, ki, ks, vi = fused_preprocess_routing(q, k, v, tau=tau, scale=scale,
                                                     int8_pv=int8_pv, block=block)
    B, _, H, D = q.shape
    vsc = r.vscale.reshape(B * H, D) if int8_pv else None
    return r.kc, r.vc, r.threshold, qi, qs, ki, ks, vi, vsc
