"""Block summaries, routing thresholds and exact-block masks (host side).

Mirrors /root/reference/_preprocess.py (``prepare``, ``_reduce_kv``,
``_compute_diag_threshold``) over the gfx950 kernels ``solattn_pool``,
``solattn_moments`` and ``solattn_route``. Every output is allocated through
the torch caching allocator on the input's device; inputs are never mutated.
"""

from __future__ import annotations

from typing import NamedTuple

import torch

from . import _capi
from ._capi import call, ptr, stream

# Reference block size (/root/reference/_preprocess.py:12); 128 is also supported.
BLOCK_SIZE = 64
# kc/vc are zero-padded to whole chunks of this many blocks
# (/root/reference/_preprocess.py:15).
GROUP_PAD = 64
HEAD_DIM = 128  # the kernels' head dim; smaller heads are zero-padded to it
SUPPORTED_BLOCKS = (64, 128)
MAX_BLOCKS = 16384  # query/key blocks per head the forward kernels accept

__all__ = ["prepare", "route", "Routing", "BLOCK_SIZE", "tau_vector"]


def tau_vector(tau, heads, device):
    """Per-head tau as the reference broadcasts it (/root/reference/_preprocess.py:18-20)."""
    return torch.full((heads,), float(tau), device=device, dtype=torch.float32)


def num_blocks(tokens: int, block: int) -> int:
    return (int(tokens) + block - 1) // block


def kernel_ready(t: torch.Tensor) -> bool:
    """Whether the kernels can read ``t`` in place: contiguous last dim, a 16-byte
    aligned base and outer strides that keep every row 16-byte aligned."""
    return (t.stride(-1) == 1 and t.data_ptr() % 16 == 0
            and all(s % 8 == 0 for s in t.stride()[:-1]))


def as_kernel_input(t: torch.Tensor) -> torch.Tensor:
    # Strided views (e.g. an interleaved qkv buffer) go in without a copy when
    # aligned; anything else is copied once, as the reference copies a
    # non-contiguous last dim (/root/reference/_tri_fwd.py:383-384).
    return t if kernel_ready(t) else t.contiguous()


def head_dim_ok(d: int) -> bool:
    """Head dims the pipelines take: multiples of 8 up to 128 (heads below 128
    run zero-padded; the padding adds exact zeros to every dot product)."""
    return 8 <= d <= HEAD_DIM and d % 8 == 0


def pad_heads(t: torch.Tensor) -> torch.Tensor:
    """A BTHD tensor with its head dim zero-padded to HEAD_DIM (on the device)."""
    if t.shape[-1] == HEAD_DIM:
        return t
    return torch.nn.functional.pad(t, (0, HEAD_DIM - t.shape[-1]))


def check_inputs(q, k, v, block: int, padded_ok: bool = True):
    if block not in SUPPORTED_BLOCKS:
        raise ValueError(f"block {block} not in {SUPPORTED_BLOCKS}")
    for name, t in (("q", q), ("k", k), ("v", v)):
        if t.device.type != "cuda":
            raise ValueError(f"{name} is not a GPU tensor")
        if t.dtype != torch.bfloat16:
            raise ValueError(f"{name} dtype {t.dtype}; the kernels are bf16-only")
        if t.dim() != 4:
            raise ValueError(f"{name} must be BTHD, got shape {tuple(t.shape)}")
    if q.shape != k.shape or k.shape != v.shape:
        raise ValueError(f"q/k/v shapes differ: {tuple(q.shape)} {tuple(k.shape)} {tuple(v.shape)}")
    if not (head_dim_ok(q.shape[-1]) if padded_ok else q.shape[-1] == HEAD_DIM):
        raise ValueError(f"head_dim {q.shape[-1]} not supported (multiples of 8 up to {HEAD_DIM}"
                         f"{'' if padded_ok else '; this entry point takes 128 only'})")
    nt = num_blocks(q.shape[1], block)
    if nt > MAX_BLOCKS:
        raise ValueError(f"{q.shape[1]} tokens make {nt} blocks of {block}; at most {MAX_BLOCKS}")
    if q.shape[1] == 0:
        raise ValueError("empty sequence")


class Routing(NamedTuple):
    """Everything the forwards consume. Layouts as in include/solattn.h."""
    kc: torch.Tensor        # bf16 [B, npad, H, D] (centred for the INT8 path)
    vc: torch.Tensor        # bf16 [B, npad, H, D]
    threshold: torch.Tensor  # fp32 [B, NT, H]
    qbar: torch.Tensor      # fp32 [B, H, NT, D]
    kc_mean: torch.Tensor   # fp32 [B, H, D]
    kc_var: torch.Tensor    # fp32 [B, H, D]
    counts: torch.Tensor    # int32 [B, H, NT] exact blocks per query block
    mask: torch.Tensor      # int32 view of uint32 [B, H, NT, ceil(NT/32)]
    vamax_part: torch.Tensor | None
    vscale: torch.Tensor | None  # fp32 [B, H, D]
    block: int
    tokens: int


def _sv(t):
    return t.stride(0), t.stride(1), t.stride(2)


def route(q, k, v, *, scale: float, tau: float, block: int = BLOCK_SIZE, int8: bool = False,
          v_absmax: bool = False, sink_blocks=(0, 0), sink_q=(0, 0)) -> Routing:
    """pool -> moments -> thresholds + routing masks, all on the device.

    ``int8`` selects the INT8 path's centred pooled keys and tau*sigma
    threshold (/root/reference/_fused_prep.py:77-81, 50-59); ``v_absmax``
    also produces the per-channel V scale from the same pass.
    """
    check_inputs(q, k, v, block)
    D0 = q.shape[-1]
    if D0 != HEAD_DIM:  # run padded, hand back the first D0 channels
        r = route(pad_heads(q), pad_heads(k), pad_heads(v), scale=scale, tau=tau, block=block,
                  int8=int8, v_absmax=v_absmax, sink_blocks=sink_blocks, sink_q=sink_q)
        cut = lambda t: None if t is None else t[..., :D0]  # noqa: E731
        return r._replace(kc=cut(r.kc), vc=cut(r.vc), qbar=cut(r.qbar), kc_mean=cut(r.kc_mean),
                          kc_var=cut(r.kc_var), vamax_part=cut(r.vamax_part),
                          vscale=cut(r.vscale))
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
    vamax = torch.empty((B, NT, H, D), **f32) if v_absmax else None
    kc_mean = torch.empty((B, H, D), **f32)
    kc_var = torch.empty((B, H, D), **f32)
    vscale = torch.empty((B, H, D), **f32) if v_absmax else None
    thr = torch.empty((B, NT, H), **f32)
    counts = torch.empty((B, H, NT), device=dev, dtype=torch.int32)
    mask = torch.empty((B, H, NT, W), device=dev, dtype=torch.int32)
    with torch.cuda.device(dev):
        s = stream(dev)
        call("solattn_pool", ptr(q), *_sv(q), ptr(k), *_sv(k), ptr(v), *_sv(v), B, T, H, D, block,
             ptr(kc), ptr(vc), npad, ptr(qbar), ptr(vamax), s)
        call("solattn_moments", ptr(kc), npad, B, NT, H, D, 1 if int8 else 0, ptr(kc_mean),
             ptr(kc_var), ptr(vamax), ptr(vscale), s)
        call("solattn_route", ptr(qbar), ptr(kc), npad, ptr(kc_mean), ptr(kc_var), B, T, H, D,
             block, float(scale), float(tau), 1 if int8 else 0, int(sink_blocks[0]),
             int(sink_blocks[1]), int(sink_q[0]), int(sink_q[1]), ptr(thr), ptr(counts),
             ptr(mask), s)
    return Routing(kc, vc, thr, qbar, kc_mean, kc_var, counts, mask, vamax, vscale, block, T)


def prepare(q, k, v, *, tau: float, scale: float, tokens: int | None = None,
            block: int = BLOCK_SIZE):
    """Returns (kc, vc, threshold); /root/reference/_preprocess.py:268-280.
    ``tokens`` is the true sequence length (q may be longer)."""
    if tokens is not None and tokens != q.shape[1]:
        q, k, v = q[:, :tokens], k[:, :tokens], v[:, :tokens]
    r = route(q, k, v, scale=scale, tau=tau, block=block)
    return r.kc, r.vc, r.threshold


_ = _capi  # the binding is loaded (or ImportError raised) on import
