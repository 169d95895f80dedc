"""Morton (Z-order) reordering of the video span for MiniMax-H3.

H3 packs one self-attention sequence: [text][cond][ref_img][ref_audio][audio][video].
Only the target video segment (contiguous, last, t-major then h then w) is
reordered; the conditioning rows keep their positions. Mirrors
/root/reference/_morton_h3.py: the video span is registered from
``PackedLayout.__init__`` and looked up by the identity of the position_ids
tensor handed to ``rope_freqs``; ``sol_h3_video_span`` is published for the
attention override's conditioning sink; hidden states and the RoPE table are
permuted together in the block-0 pre-hook and restored after the last block.

Each permutation is one gather of all S rows through a composed index
(identity outside the span, ``start + perm`` inside) on the gfx950 reorder
kernel, instead of a clone plus a fancy-indexed copy.
"""

from __future__ import annotations

import logging
import sys

import torch

from ._morton import morton_perm, reorder_tokens

_INSTALLED: set = set()
_PATCHED_LAYOUTS: set = set()
# The kernels block from absolute row 0; the span is rotated onto this grid.
BLOCK_SIZE = 64
_DEVICE_CACHE: dict = {}
# id(position_ids) -> (layout, bounds, span); the layout is kept alive so the id
# cannot be recycled underneath the lookup.
_SPANS: dict = {}

__all__ = ["install_h3_morton", "install_h3_hooks"]


def _perm_for(grid, curve, device, start, block=None):
    """Morton permutation for a video span starting at absolute row ``start``,
    rotated by the span's misalignment to the block grid so Z-order cells are
    not split across blocks (/root/reference/_morton_h3.py:42-61)."""
    block = BLOCK_SIZE if block is None else int(block)
    pad = (-int(start)) % block
    return morton_perm(grid, device, curve, roll=pad)


def _composed(grid, curve, device, start, stop, total, block=None):
    """(forward, inverse) row indices over all ``total`` rows."""
    block = BLOCK_SIZE if block is None else int(block)
    key = (tuple(grid), curve, str(device), int(start), int(stop), int(total), block)
    hit = _DEVICE_CACHE.get(key)
    if hit is None:
        perm, inverse = _perm_for(grid, curve, device, start, block)
        fwd = torch.arange(total, device=device, dtype=torch.int64)
        inv = fwd.clone()
        fwd[start:stop] = perm + start
        inv[start:stop] = inverse + start
        hit = (fwd, inv)
        _DEVICE_CACHE[key] = hit
    return hit


def _video_span(layout, latent_t, latent_h, latent_w):
    """(start, stop, grid) of the target video segment, or None
    (/root/reference/_morton_h3.py:64-82)."""
    segments = getattr(layout, "segments", None)
    if not segments:
        return None
    span = next(((a, b) for a, b, kind in segments if kind == "video"), None)
    if span is None:
        return None
    start, stop = span
    grid = (int(latent_t), int(latent_h) // 2, int(latent_w) // 2)
    if grid[0] * grid[1] * grid[2] != stop - start:
        logging.info(f"[sol_attn] H3 Morton skipped: video segment {stop - start} rows "
                     f"does not match grid {grid}")
        return None
    return start, stop, grid


def _patch_packed_layout(module):
    """Register the video span of every PackedLayout built, without mutating it."""
    layout_cls = getattr(module, "PackedLayout", None)
    if layout_cls is None:
        raise RuntimeError(f"{module.__name__} has no PackedLayout")
    if id(layout_cls) in _PATCHED_LAYOUTS:
        return
    original_init = layout_cls.__init__

    def __init__(self, text_len, latent_t, latent_h, latent_w, audio_t, *args, **kwargs):
        original_init(self, text_len, latent_t, latent_h, latent_w, audio_t, *args, **kwargs)
        try:
            span = _video_span(self, latent_t, latent_h, latent_w)
        except Exception as exc:  # never break model construction
            logging.info(f"[sol_attn] H3 Morton span resolution failed: {exc}")
            span = None
        bounds = next(((a, b) for a, b, kind in getattr(self, "segments", []) or []
                       if kind == "video"), None)
        if torch.is_tensor(getattr(self, "position_ids", None)) and bounds is not None:
            _SPANS[id(self.position_ids)] = (self, bounds, span)

    layout_cls.__init__ = __init__
    _PATCHED_LAYOUTS.add(id(layout_cls))


_logged: set = set()


def _log_once(message):
    if message not in _logged:
        _logged.add(message)
        logging.info(f"[sol_attn] H3 Morton: {message}")


def install_h3_morton(model, block=None):
    """Idempotently install the reorder (/root/reference/_morton_h3.py:110-226).
    Inert without transformer_options['sol_morton']; always publishes the video
    span for the conditioning sink."""
    if id(model) in _INSTALLED:
        return
    for attr in ("rope_freqs", "_forward", "blocks"):
        if not hasattr(model, attr):
            raise RuntimeError(f"MiniMax-H3 Morton needs .{attr} on the diffusion model")

    _patch_packed_layout(sys.modules[type(model).__module__])

    original_forward = model._forward
    original_rope_freqs = model.rope_freqs

    def _forward(x, timestep, context, transformer_options={}, **kwargs):
        previous = getattr(model, "_sol_morton_active", False)
        model._sol_morton_active = bool(transformer_options.get("sol_morton"))
        model._sol_morton_curve = transformer_options.get("sol_morton_curve", "3d")
        model._sol_morton_block = transformer_options.get("sol_block_size", block)
        model._sol_transformer_options = transformer_options
        try:
            return original_forward(x, timestep, context,
                                    transformer_options=transformer_options, **kwargs)
        finally:
            model._sol_morton_active = previous
            model._sol_morton_span = None
            model._sol_morton_state = None
            model._sol_transformer_options = None
            transformer_options.pop("sol_h3_video_span", None)

    def rope_freqs(position_ids, device):
        """Publish the layout only; permuting happens in the block hook."""
        model._sol_morton_span = None
        model._sol_morton_state = None
        entry = _SPANS.get(id(position_ids))
        if entry is None:
            _log_once("no layout registered; Morton and the conditioning sink are inactive")
            return original_rope_freqs(position_ids, device)
        _layout, bounds, span = entry
        options = getattr(model, "_sol_transformer_options", None)
        if options is not None:
            options["sol_h3_video_span"] = bounds
        if getattr(model, "_sol_morton_active", False):
            if span is None:
                _log_once("video grid does not match the segment; Morton inactive")
            else:
                model._sol_morton_span = span
        return original_rope_freqs(position_ids, device)

    def pre_hook(module, args):
        # Blocks are called as block(h, t_emb, mod_segments, rope_freqs, ...).
        if len(args) < 4:
            return None
        if module is not first:
            state = getattr(model, "_sol_morton_state", None)
            if state is None:
                return None
            return args[:3] + (state[1],) + tuple(args[4:])
        model._sol_morton_state = None
        span = getattr(model, "_sol_morton_span", None)
        if span is None:
            return None
        start, stop, grid = span
        h, rope = args[0], args[3]
        if not torch.is_tensor(h) or h.ndim != 2 or h.shape[0] < stop:
            _log_once(f"hidden states do not cover the video span {(start, stop)}; inactive")
            return None
        if not torch.is_tensor(rope) or rope.ndim < 2 or rope.shape[1] != h.shape[0]:
            _log_once(f"rope table {tuple(rope.shape) if torch.is_tensor(rope) else type(rope)} "
                      f"does not match {h.shape[0]} tokens; inactive")
            return None
        curve = getattr(model, "_sol_morton_curve", "3d")
        fwd, inv = _composed(grid, curve, h.device, start, stop, h.shape[0],
                             getattr(model, "_sol_morton_block", None))
        h = reorder_tokens(h, fwd, dim=0)
        # The rotation table is elementwise per row, so permuting it equals
        # permuting position_ids.
        rope = reorder_tokens(rope, fwd.to(rope.device), dim=1)
        model._sol_morton_state = (inv, rope)
        return (h,) + args[1:3] + (rope,) + tuple(args[4:])

    def post_hook(_module, _args, output):
        state = getattr(model, "_sol_morton_state", None)
        span = getattr(model, "_sol_morton_span", None)
        model._sol_morton_state = None
        if state is None or span is None:
            return None
        _start, stop, _grid = span
        inv, _rope = state
        if not torch.is_tensor(output) or output.shape[0] < stop or output.shape[0] != inv.numel():
            logging.error("[sol_attn] H3 Morton: block stack changed the token count "
                          f"({tuple(output.shape) if torch.is_tensor(output) else type(output)}); "
                          "cannot restore order")
            return None
        return reorder_tokens(output, inv, dim=0)

    first = model.blocks[0]
    model._forward = _forward
    model.rope_freqs = rope_freqs
    for blk in model.blocks:
        blk.register_forward_pre_hook(pre_hook)
    model.blocks[-1].register_forward_hook(post_hook)
    _INSTALLED.add(id(model))


install_h3_hooks = install_h3_morton
