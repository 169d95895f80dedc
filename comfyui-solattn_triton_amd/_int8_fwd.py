"""INT8 Sol-Attn forward (host side).

Mirrors ``sol_attn_int8`` of /root/reference/_int8_fwd.py:379-432:
``solattn_sol_attn_int8`` runs pool -> moments (centred) -> route (tau*sigma)
-> quant (Q, smoothed K, per-channel V) -> fwd_int8 in one call. The exact
branch's QK runs on int8 MFMA; P.V runs on int8 MFMA with ``int8_pv`` and in
bf16 otherwise. ``use_tma`` is accepted and ignored.
"""

from __future__ import annotations

import torch

from ._capi import QUANT_BLOCK, call, ptr, stream
from ._preprocess import BLOCK_SIZE, Routing, as_kernel_input, check_inputs
from ._tri_fwd import _workspace

BLOCK = BLOCK_SIZE
# How the int8 P.V forms its P codes (int8_pv=True): against each routed
# block's row max (the reference's arithmetic), or against the row's running
# max with int32 sums across blocks (SOLATTN_PV_INT8_RUNNING: no per-block
# conversion; coarser codes for blocks below the running max).
PV_CODES = ("block", "running")

__all__ = ["sol_attn_int8", "forward_int8", "PV_CODES"]


def _pv_mode(int8_pv, pv_codes) -> int:
    """The C ABI's int8_pv value: SOLATTN_PV_BF16 (0), SOLATTN_PV_INT8 (1) or
    SOLATTN_PV_INT8_RUNNING (2)."""
    if pv_codes not in PV_CODES:
        raise ValueError(f"pv_codes must be one of {PV_CODES}, got {pv_codes!r}")
    if not int8_pv:
        return 0
    return 2 if pv_codes == "running" else 1


def sol_attn_int8(q, k, v, *, scale=None, tau=1.0, sink_blocks=(0, 0), sink_q=(0, 0),
                  use_tma=False, int8_pv=True, block=BLOCK, quant_block=None, pv_codes="block"):
    """Sol-Attn with an INT8 exact branch. Same contract as ``sol_attn``.
    ``quant_block=128`` quantises Q and smoothed K with one scale per 128-token
    block instead of per token (an option of this build, BASELINE config 3's
    wording; the default is the reference's per-token rule). ``pv_codes``
    (with ``int8_pv``): "block" quantises P against each routed block's row
    max, as the reference; "running" against the row's running max."""
    if quant_block not in (None, QUANT_BLOCK):
        raise ValueError(f"quant_block must be None or {QUANT_BLOCK}, got {quant_block}")
    mode = _pv_mode(int8_pv, pv_codes)
    check_inputs(q, k, v, block)
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    q, k, v = as_kernel_input(q), as_kernel_input(k), as_kernel_input(v)
    B, T, H, D = q.shape
    out = torch.empty((B, T, H, D), device=q.device, dtype=torch.bfloat16)
    ws = _workspace(q, block, True)
    with torch.cuda.device(q.device):
        call("solattn_sol_attn_int8" if quant_block is None else "solattn_sol_attn_int8_qblock",
             ptr(q), q.stride(0), q.stride(1), q.stride(2), ptr(k),
             k.stride(0), k.stride(1), k.stride(2), ptr(v), v.stride(0), v.stride(1), v.stride(2),
             B, T, H, D, block, float(scale), float(tau), int(sink_blocks[0]), int(sink_blocks[1]),
             int(sink_q[0]), int(sink_q[1]), mode, ptr(ws), ws.numel(), ptr(out),
             out.stride(0), out.stride(1), out.stride(2), stream(q.device))
    return out


def forward_int8(q, v, routing: Routing, qi, qs, ki, ks, vi=None, *, scale=None, int8_pv=True,
                 out=None, pv_codes="block"):
    """The INT8 forward kernel alone (head dim 128), on the outputs of
    ``fused_preprocess_routing``."""
    mode = _pv_mode(int8_pv, pv_codes)
    check_inputs(q, q, q, routing.block, padded_ok=False)
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    q, v = as_kernel_input(q), as_kernel_input(v)
    B, T, H, D = q.shape
    if out is None:
        out = torch.empty((B, T, H, D), device=q.device, dtype=torch.bfloat16)
    npad = routing.kc.shape[1]
    TP = qi.shape[1]
    with torch.cuda.device(q.device):
        call("solattn_fwd_int8", ptr(q), q.stride(0), q.stride(1), q.stride(2), ptr(qi), ptr(qs),
             ptr(ki), ptr(ks), ptr(vi if int8_pv else None),
             ptr(routing.vscale if int8_pv else None), ptr(v), v.stride(0), v.stride(1),
             v.stride(2), TP, ptr(routing.kc), ptr(routing.vc), npad, ptr(routing.counts),
             ptr(routing.mask), B, T, H, D, routing.block, float(scale),
             mode, ptr(out), out.stride(0), out.stride(1), out.stride(2),
             stream(q.device))
    return out
