"""BF16 Sol-Attn forward (host side).

Mirrors ``sol_attn`` of /root/reference/_tri_fwd.py:354-410 over the gfx950
library: ``solattn_sol_attn`` runs pool -> moments -> route -> fwd_bf16 in one
call on a workspace from the torch caching allocator. ``use_tma`` is accepted
and ignored (the descriptor kernels are an NVIDIA TMA feature).
"""

from __future__ import annotations

import torch

from ._capi import LIB, call, ptr, stream
from ._preprocess import BLOCK_SIZE, Routing, as_kernel_input, check_inputs

BLOCK = BLOCK_SIZE
GROUP = 32  # the reference's group width; kept for API compatibility only

__all__ = ["sol_attn", "forward_bf16", "BLOCK"]


def _has_tma(device):
    """The reference's TMA probe (/root/reference/_tri_fwd.py:28-39). There are no
    descriptor kernels on gfx950, so this is always False."""
    return False


def _workspace(q, block: int, int8: bool) -> torch.Tensor:
    B, T, H, D = q.shape
    nbytes = LIB.solattn_sol_attn_workspace_bytes(B, T, H, D, block, 1 if int8 else 0)
    return torch.empty(nbytes, device=q.device, dtype=torch.uint8)


def sol_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, *, scale: float | None = None,
             tau: float = 1.0, sink_blocks: tuple = (0, 0), sink_q: tuple = (0, 0),
             use_tma: bool = False, block: int = BLOCK) -> torch.Tensor:
    """Run Sol-Attn on BTHD bf16 inputs; returns a fresh BTHD bf16 tensor.

    Head dims below 128 (multiples of 8) run zero-padded to 128 inside the
    library call. Each query block attends exactly to its routed blocks (score above the
    Gaussian threshold mu + tau*sigma, the diagonal band |i-j| <= 1 and the
    ``sink_blocks`` KV range) and to one pooled key/value per remaining block;
    query blocks inside ``sink_q`` attend everything exactly.
    """
    check_inputs(q, k, v, block)
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    q, k, v = as_kernel_input(q), as_kernel_input(k), as_kernel_input(v)
    B, T, H, D = q.shape
    out = torch.empty((B, T, H, D), device=q.device, dtype=torch.bfloat16)
    ws = _workspace(q, block, False)
    with torch.cuda.device(q.device):
        call("solattn_sol_attn", ptr(q), q.stride(0), q.stride(1), q.stride(2), ptr(k), k.stride(0),
             k.stride(1), k.stride(2), ptr(v), v.stride(0), v.stride(1), v.stride(2), B, T, H, D,
             block, float(scale), float(tau), int(sink_blocks[0]), int(sink_blocks[1]),
             int(sink_q[0]), int(sink_q[1]), ptr(ws), ws.numel(), ptr(out), out.stride(0),
             out.stride(1), out.stride(2), stream(q.device))
    return out


def forward_bf16(q, k, v, routing: Routing, *, scale: float | None = None,
                 out: torch.Tensor | None = None) -> torch.Tensor:
    """The forward kernel alone (head dim 128), on routing produced by
    ``_preprocess.route``."""
    check_inputs(q, k, v, routing.block, padded_ok=False)
    scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
    q, k, v = as_kernel_input(q), as_kernel_input(k), as_kernel_input(v)
    B, T, H, D = q.shape
    if out is None:
        out = torch.empty((B, T, H, D), device=q.device, dtype=torch.bfloat16)
    npad = routing.kc.shape[1]
    with torch.cuda.device(q.device):
        call("solattn_fwd_bf16", ptr(q), q.stride(0), q.stride(1), q.stride(2), ptr(k), k.stride(0),
             k.stride(1), k.stride(2), ptr(v), v.stride(0), v.stride(1), v.stride(2),
             ptr(routing.kc), ptr(routing.vc), npad, ptr(routing.counts), ptr(routing.mask),
             B, T, H, D, routing.block, float(scale), ptr(out), out.stride(0),
             out.stride(1), out.stride(2), stream(q.device))
    return out
