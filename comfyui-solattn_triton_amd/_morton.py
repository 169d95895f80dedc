"""Morton (Z-order) token reordering and the Wan integration hooks.

Video latents are laid out frame-major, then row-major, so a block of tokens is
a thin strip of one frame. Z-ordering makes each block a compact 3-D
neighbourhood, which concentrates attention mass into fewer blocks. The
permutation is applied once before the block stack and inverted after it, with
the RoPE table permuted to match, so it is a no-op for dense attention.

Mirrors /root/reference/_morton.py. The permutation is computed once per grid
on the host (``solattn_morton_perm``) and cached on the device (the reference
copies it to the device on every call, :73); the row gathers run on the gfx950
``solattn_reorder_rows`` kernel instead of ``index_select``.

The permute-or-not decision is made in exactly one place, the block-0
pre-hook, which sees the hidden states and the RoPE table together
(/root/reference/_morton.py:13-19): deciding for the positions and the tokens
in separate places corrupts the output whenever the two guards disagree.
"""

from __future__ import annotations

import ctypes
import logging
import math
import weakref

import torch

from ._capi import LIB, SolAttnError, call, ptr, stream

_PERM_CACHE: dict = {}

__all__ = ["morton_perm", "reorder_tokens", "install_wan_morton"]

_CURVES = {"3d": 0, "2d_frame": 1}


def _host_perm(grid, curve: str, roll: int):
    key = (tuple(int(g) for g in grid), curve, int(roll))
    hit = _PERM_CACHE.get(key)
    if hit is None:
        if curve not in _CURVES:
            raise ValueError(f"unknown Morton curve {curve!r}; use one of {sorted(_CURVES)}")
        frames, height, width = key[0]
        n = frames * height * width
        perm = torch.empty(n, dtype=torch.int64)
        inverse = torch.empty(n, dtype=torch.int64)
        rc = LIB.solattn_morton_perm(frames, height, width, _CURVES[curve], int(roll),
                                     ctypes.c_void_p(perm.data_ptr()),
                                     ctypes.c_void_p(inverse.data_ptr()))
        if rc != 0:
            raise SolAttnError(f"solattn_morton_perm failed ({rc}): "
                               f"{LIB.solattn_last_error().decode(errors='replace')}")
        hit = {"cpu": (perm, inverse)}
        _PERM_CACHE[key] = hit
    return hit


def morton_perm(grid, device, curve: str = "3d", roll: int = 0):
    """Z-order permutation of a (frames, height, width) grid and its inverse,
    int64 on ``device``. ``curve="2d_frame"`` keeps frames in order and
    Z-orders within each. ``roll`` rotates the permutation (torch.roll) before
    the inverse is taken (/root/reference/_morton_h3.py:50-53)."""
    hit = _host_perm(grid, curve, roll)
    dev = torch.device(device)
    dkey = str(dev)
    if dkey not in hit:
        perm, inverse = hit["cpu"]
        hit[dkey] = (perm.to(dev), inverse.to(dev))
    return hit[dkey]


def reorder_tokens(x: torch.Tensor, index: torch.Tensor, dim: int = 1) -> torch.Tensor:
    """``x.index_select(dim, index)`` for dim 0 or 1 on the gather kernel.

    The dims after ``dim`` form one contiguous row; a tensor whose rows are not
    16-byte aligned is made contiguous first.
    """
    if dim not in (0, 1) or x.dim() <= dim:
        raise ValueError(f"reorder_tokens gathers along dim 0 or 1, got dim={dim} for {tuple(x.shape)}")
    if x.device.type != "cuda":
        raise ValueError("reorder_tokens needs a GPU tensor")
    isz = x.element_size()
    inner = math.prod(x.shape[dim + 1:])
    row_bytes = inner * isz

    def fits(t):
        inner_contig = t[(0,) * (dim + 1)].is_contiguous() if t.numel() else True
        outer_ok = dim == 0 or (t.stride(0) * isz) % 16 == 0
        return (inner_contig and row_bytes % 16 == 0 and (t.stride(dim) * isz) % 16 == 0
                and outer_ok and t.data_ptr() % 16 == 0)

    if not fits(x):
        x = x.contiguous()
        if not fits(x):
            raise ValueError(f"rows of {row_bytes} bytes are not a multiple of 16")
    index = index.to(device=x.device, dtype=torch.int64).contiguous()
    shape = list(x.shape)
    shape[dim] = index.numel()
    out = torch.empty(shape, device=x.device, dtype=x.dtype)
    if out.numel() == 0:
        return out
    batch = 1 if dim == 0 else x.shape[0]
    with torch.cuda.device(x.device):
        call("solattn_reorder_rows", ptr(x), x.shape[dim], x.stride(0) * isz if dim == 1 else 0,
             x.stride(dim) * isz, ptr(out), out.stride(0) * isz if dim == 1 else 0,
             out.stride(dim) * isz, batch, index.numel(), row_bytes, ptr(index),
             stream(x.device))
    return out


def _gather(x: torch.Tensor, index: torch.Tensor, dim: int) -> torch.Tensor:
    """The hooks' row permutation: the gfx950 gather kernel for GPU tensors;
    a pass whose tensors live on the host (no kernel can touch them) is
    permuted with ``index_select``, as the reference does on any device."""
    if x.device.type != "cuda":
        return x.index_select(dim, index.to(x.device))
    return reorder_tokens(x, index, dim=dim)


class _WanReorder:
    """Reorder state of one Wan-style model for one forward pass.

    The block-0 pre-hook is the only place that decides (it holds the hidden
    states and the RoPE table together): if the tokens are exactly the video
    grid, both are permuted there, later blocks get the permuted table, and the
    last block's output is put back in raster order. Any mismatch (reference
    latents prepended, context latents appended) leaves the pass untouched.
    """

    installed = weakref.WeakSet()  # models with the hooks

    def __init__(self, model):
        self.first = model.blocks[0]
        self.inverse = None  # set while a permuted pass is in flight
        self.freqs = None

    def _plan(self, x, freqs, options):
        """(perm, inverse) when this pass can be reordered, else None (logged once)."""
        grid = options.get("grid_sizes")
        if grid is None:
            _log_once("transformer_options has no grid_sizes; inactive")
            return None
        tokens = math.prod(int(g) for g in grid)
        if not (torch.is_tensor(x) and x.ndim == 3 and x.shape[1] == tokens):
            shape = tuple(x.shape) if torch.is_tensor(x) else type(x).__name__
            _log_once(f"token count {shape} != video grid {tuple(grid)} ({tokens}); "
                      "reference/context streams present, inactive")
            return None
        if not (torch.is_tensor(freqs) and freqs.ndim >= 2 and freqs.shape[1] == tokens):
            shape = tuple(freqs.shape) if torch.is_tensor(freqs) else type(freqs).__name__
            _log_once(f"rope table {shape} does not match the video grid ({tokens}); inactive")
            return None
        return morton_perm(grid, x.device, options.get("sol_morton_curve", "3d"))

    def before_block(self, module, args, kwargs):
        options = kwargs.get("transformer_options") or {}
        if module is self.first:
            self.inverse = self.freqs = None
            if not options.get("sol_morton") or not args:
                return None
            plan = self._plan(args[0], kwargs.get("freqs"), options)
            if plan is None:
                return None
            perm, self.inverse = plan
            self.freqs = _gather(kwargs["freqs"], perm, 1)
            return (_gather(args[0], perm, 1),) + tuple(args[1:]), {**kwargs, "freqs": self.freqs}
        if self.inverse is None:
            return None
        # hidden states are already in Morton order; only the table is swapped in
        return tuple(args), {**kwargs, "freqs": self.freqs}

    def after_stack(self, _module, _args, _kwargs, output):
        inverse, self.inverse, self.freqs = self.inverse, None, None
        if inverse is None:
            return None
        if not (torch.is_tensor(output) and output.ndim >= 2 and output.shape[1] == inverse.numel()):
            shape = tuple(output.shape) if torch.is_tensor(output) else type(output).__name__
            logging.error(f"[sol_attn] Wan Morton: block stack changed the token count ({shape}); "
                          "cannot restore order")
            return None
        return _gather(output, inverse, 1)


_logged: set = set()


def _log_once(message):
    if message not in _logged:
        _logged.add(message)
        logging.info(f"[sol_attn] Wan Morton: {message}")


def install_wan_morton(diffusion_model):
    """Install the reorder hooks on a Wan-style model, once per model
    (/root/reference/_morton.py:85-153). Inert unless
    transformer_options["sol_morton"] is set for the pass."""
    if diffusion_model in _WanReorder.installed:
        return
    if not hasattr(diffusion_model, "blocks"):
        raise RuntimeError("Morton reordering needs .blocks on the diffusion model")
    state = _WanReorder(diffusion_model)
    for block in diffusion_model.blocks:
        block.register_forward_pre_hook(state.before_block, with_kwargs=True)
    diffusion_model.blocks[-1].register_forward_hook(state.after_stack, with_kwargs=True)
    _WanReorder.installed.add(diffusion_model)
