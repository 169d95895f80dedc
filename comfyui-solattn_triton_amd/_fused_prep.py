"""Fused preprocess for the INT8 path (host side).

Mirrors /root/reference/_fused_prep.py:62-98: pooled keys centred by their own
mean (K smoothing), thresholds tau*sigma, per-token INT8 Q and smoothed K,
per-channel INT8 V, all from the gfx950 kernels.
"""

from __future__ import annotations

import torch

from ._capi import QUANT_BLOCK, call, ptr, stream
from ._preprocess import BLOCK_SIZE, HEAD_DIM, Routing, as_kernel_input, pad_heads, route

__all__ = ["fused_preprocess", "fused_preprocess_routing"]


def fused_preprocess_routing(q, k, v, *, tau, scale, int8_pv=True, block=BLOCK_SIZE,
                             sink_blocks=(0, 0), sink_q=(0, 0), quant_block=None):
    """(Routing, qi, qs, ki, ks, vi) -- the INT8 path's inputs to the forward.
    Head dims below 128 run zero-padded; codes come back for the first D
    channels (the padded ones are 0). ``quant_block=128``: Q and K scales per
    128-token block (written for every token), as ``sol_attn_int8``."""
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
