"""Per-token and per-channel INT8 quantisation (host side).

Mirrors /root/reference/_fused_quant.py (``quantize_bthd``,
``quantize_v_per_channel``) over ``solattn_quant_rows`` / ``solattn_quant_v``.
Codes: round half away from zero, clamped to [-127, 127]; scales
max|x| / 127 floored at 1e-8.
"""

from __future__ import annotations

import torch

from ._capi import call, ptr, stream
from ._preprocess import HEAD_DIM, as_kernel_input, head_dim_ok, pad_heads

__all__ = ["quantize_bthd", "quantize_v_per_channel"]


def _check(x):
    if x.device.type != "cuda" or x.dtype != torch.bfloat16 or x.dim() != 4 or \
            not head_dim_ok(x.shape[-1]):
        raise ValueError(f"expected a bf16 GPU BTHD tensor with a head_dim of 8..{HEAD_DIM} "
                         f"(multiple of 8), got {x.dtype} {tuple(x.shape)} on {x.device}")


def quantize_bthd(x, mean=None, rows=16, num_warps=4, out_rows=None):
    """(xi int8 [B, TP, H, D], xs fp32 [B, TP, H]); ``mean`` [B*H, D] smooths x
    first. ``rows`` / ``num_warps`` are the reference's launch knobs, accepted
    and unused. /root/reference/_fused_quant.py:45-58."""
    _check(x)
    D0 = x.shape[-1]
    if D0 != HEAD_DIM:  # padded channels are 0 after smoothing by a 0 mean: same row max
        if mean is not None:
            mean = torch.nn.functional.pad(mean.reshape(-1, D0).float(), (0, HEAD_DIM - D0))
        xi, xs = quantize_bthd(pad_heads(x), mean=mean, out_rows=out_rows)
        return xi[..., :D0], xs
    x = as_kernel_input(x)
    B, T, H, D = x.shape
    TP = T if out_rows is None else int(out_rows)
    xi = torch.empty((B, TP, H, D), device=x.device, dtype=torch.int8)
    xs = torch.empty((B, TP, H), device=x.device, dtype=torch.float32)
    if mean is not None:
        mean = mean.to(device=x.device, dtype=torch.float32).contiguous()
        if mean.numel() != B * H * D:
            raise ValueError(f"mean must hold B*H*D = {B * H * D} values")
    with torch.cuda.device(x.device):
        call("solattn_quant_rows", ptr(x), x.stride(0), x.stride(1), x.stride(2), B, T, H, D,
             ptr(mean), ptr(xi), ptr(xs), TP, stream(x.device))
    return xi, xs


def quantize_v_per_channel(v, rows=16, num_warps=4, out_rows=None, absmax=None):
    """INT8 V with one scale per (batch, head, channel): returns (vi, scale
    [B*H, D]). /root/reference/_fused_quant.py:91-113. ``absmax`` [B, H, D]
    comes from a pass that already read V (the pooling pass does)."""
    _check(v)
    D0 = v.shape[-1]
    if D0 != HEAD_DIM:  # padded channels: absmax 0 -> scale 1e-8, codes 0
        vi, scale = quantize_v_per_channel(pad_heads(v), out_rows=out_rows,
                                           absmax=None if absmax is None else
                                           torch.nn.functional.pad(absmax, (0, HEAD_DIM - D0)))
        return vi[..., :D0], scale[:, :D0]
    v = as_kernel_input(v)
    B, T, H, D = v.shape
    TP = T if out_rows is None else int(out_rows)
    if absmax is None:
        absmax = v.abs().amax(dim=1)
    scale = absmax.float().div(127.0).clamp_min_(1e-8).reshape(B * H, D).contiguous()
    vi = torch.empty((B, TP, H, D), device=v.device, dtype=torch.int8)
    with torch.cuda.device(v.device):
        call("solattn_quant_v", ptr(v), v.stride(0), v.stride(1), v.stride(2), B, T, H, D,
             ptr(scale), ptr(vi), TP, stream(v.device))
    return vi, scale
