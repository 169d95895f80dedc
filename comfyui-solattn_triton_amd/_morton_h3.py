"""Morton (Z-order) reordering of MiniMax-H3's video span.

H3 packs one self-attention sequence: [text][cond][ref_img][ref_audio][audio]
[video]. Only the target video segment (contiguous, last, t-major then h then
w) is reordered; conditioning rows keep their places. Behaviour of
/root/reference/_morton_h3.py:

* every ``PackedLayout`` built registers its video segment, keyed by its
  position_ids tensor (the layout class's constructor is wrapped, since model
  revisions build layouts in different places);
* ``rope_freqs(position_ids, device)`` looks the segment up and publishes its
  bounds as transformer_options['sol_h3_video_span'] (the attention override's
  conditioning sink needs it whether or not tokens are reordered);
* the block-0 pre-hook is the single decision point: it permutes the hidden
  states and the RoPE table together, later blocks get the permuted table,
  and the last block's output is restored.

The permutation is rotated by the span's misalignment to the routing block
grid ((-start) % block), so Z-order cells are not split across blocks; the few
rows it displaces land in the block shared with the conditioning rows, which
the exact-KV sink keeps exact. Each permutation is a single gather of all S
rows through a composed index (identity outside the span, ``start + perm``
inside) on the gfx950 reorder kernel.
"""

from __future__ import annotations

import logging
import sys
import weakref

import torch

from ._morton import morton_perm, reorder_tokens

# The kernels block from absolute row 0; the span is rotated onto this grid.
BLOCK_SIZE = 64

__all__ = ["install_h3_morton", "install_h3_hooks"]

_logged: set = set()


def _log_once(message):
    if message not in _logged:
        _logged.add(message)
        logging.info(f"[sol_attn] H3 Morton: {message}")


def _gather(x: torch.Tensor, index: torch.Tensor, dim: int) -> torch.Tensor:
    """The hooks' row permutation: the gfx950 gather kernel for GPU tensors;
    a pass whose tensors live on the host (no kernel can touch them) is
    permuted with ``index_select``, as the reference does on any device."""
    if x.device.type != "cuda":
        return x.index_select(dim, index.to(x.device))
    return reorder_tokens(x, index, dim=dim)


# ------------------------------------------------------------ span registry
def _video_bounds(layout):
    """(start, stop) of the layout's 'video' segment, or None."""
    for start, stop, kind in getattr(layout, "segments", None) or ():
        if kind == "video":
            return start, stop
    return None


def _video_span(layout, latent_t, latent_h, latent_w):
    """(start, stop, grid) of the target video segment when its row count is
    the patchified latent grid (t, h/2, w/2), else None."""
    bounds = _video_bounds(layout)
    if bounds is None:
        return None
    grid = (int(latent_t), int(latent_h) // 2, int(latent_w) // 2)
    rows = bounds[1] - bounds[0]
    if grid[0] * grid[1] * grid[2] != rows:
        logging.info(f"[sol_attn] H3 Morton skipped: video segment {rows} rows "
                     f"does not match grid {grid}")
        return None
    return bounds[0], bounds[1], grid


class _SpanRegistry:
    """Video spans of the layouts built so far, keyed by their position_ids.

    An entry holds a weak reference to its position_ids tensor and is only
    returned for that very tensor, so a recycled id never matches a stale
    entry; entries of freed tensors are dropped as new ones arrive."""

    def __init__(self):
        self._entries: dict = {}
        self._wrapped = weakref.WeakSet()  # layout classes already wrapped

    def register(self, layout, latent_t, latent_h, latent_w):
        position_ids = getattr(layout, "position_ids", None)
        bounds = _video_bounds(layout)
        if not torch.is_tensor(position_ids) or bounds is None:
            return
        try:
            span = _video_span(layout, latent_t, latent_h, latent_w)
        except Exception as exc:  # never break model construction
            logging.info(f"[sol_attn] H3 Morton span resolution failed: {exc}")
            span = None
        self._entries = {key: e for key, e in self._entries.items() if e[0]() is not None}
        self._entries[id(position_ids)] = (weakref.ref(position_ids), bounds, span)

    def lookup(self, position_ids):
        """(bounds, span or None) for this position_ids tensor, or None."""
        entry = self._entries.get(id(position_ids))
        if entry is None or entry[0]() is not position_ids:
            return None
        return entry[1], entry[2]

    def watch(self, module):
        """Wrap ``module.PackedLayout.__init__`` (once) so every layout registers."""
        layout_cls = getattr(module, "PackedLayout", None)
        if layout_cls is None:
            raise RuntimeError(f"{module.__name__} has no PackedLayout")
        if layout_cls in self._wrapped:
            return
        build = layout_cls.__init__
        registry = self

        def __init__(self, text_len, latent_t, latent_h, latent_w, audio_t, *args, **kwargs):
            build(self, text_len, latent_t, latent_h, latent_w, audio_t, *args, **kwargs)
            registry.register(self, latent_t, latent_h, latent_w)

        layout_cls.__init__ = __init__
        self._wrapped.add(layout_cls)


_SPANS = _SpanRegistry()
_INDEX_CACHE: dict = {}


def _composed(grid, curve, device, start, stop, total, block=None):
    """(forward, inverse) row indices over all ``total`` rows: the rotated
    Morton permutation of rows [start, stop), identity elsewhere."""
    block = BLOCK_SIZE if block is None else int(block)
    key = (tuple(grid), curve, str(device), int(start), int(stop), int(total), block)
    hit = _INDEX_CACHE.get(key)
    if hit is None:
        perm, inverse = morton_perm(grid, device, curve, roll=(-int(start)) % block)
        forward = torch.arange(total, device=device, dtype=torch.int64)
        backward = forward.clone()
        forward[start:stop] = perm + start
        backward[start:stop] = inverse + start
        hit = _INDEX_CACHE[key] = (forward, backward)
    return hit


# ------------------------------------------------------------ model hooks
class _H3Reorder:
    """Per-model state across one forward pass."""

    installed = weakref.WeakSet()  # models with the hooks

    def __init__(self, model, block):
        self.first = model.blocks[0]
        self.default_block = block
        self.active = False      # sol_morton set for the running pass
        self.curve = "3d"
        self.block = block
        self.options = None      # the running pass's transformer_options
        self.span = None         # (start, stop, grid) once rope_freqs resolved it
        self.inverse = None      # composed inverse index while permuted
        self.rope = None         # permuted RoPE table while permuted

    def _clear_pass(self):
        self.span = self.inverse = self.rope = None

    def wrap_forward(self, original):
        def _forward(x, timestep, context, transformer_options={}, **kwargs):
            saved = self.active
            self.active = bool(transformer_options.get("sol_morton"))
            self.curve = transformer_options.get("sol_morton_curve", "3d")
            self.block = transformer_options.get("sol_block_size", self.default_block)
            self.options = transformer_options
            try:
                return original(x, timestep, context, transformer_options=transformer_options,
                                **kwargs)
            finally:
                self.active = saved
                self.options = None
                self._clear_pass()
                transformer_options.pop("sol_h3_video_span", None)
        return _forward

    def wrap_rope(self, original):
        def rope_freqs(position_ids, device):
            """Publish the layout; permuting is left to the block-0 hook."""
            self._clear_pass()
            found = _SPANS.lookup(position_ids)
            if found is None:
                _log_once("no layout registered; Morton and the conditioning sink are inactive")
                return original(position_ids, device)
            bounds, span = found
            if self.options is not None:
                self.options["sol_h3_video_span"] = bounds
            if self.active:
                if span is None:
                    _log_once("video grid does not match the segment; Morton inactive")
                self.span = span
            return original(position_ids, device)
        return rope_freqs

    def before_block(self, module, args):
        # blocks are called as block(h, t_emb, mod_segments, rope, ...)
        if len(args) < 4:
            return None
        if module is not self.first:
            if self.inverse is None:
                return None
            return tuple(args[:3]) + (self.rope,) + tuple(args[4:])
        self.inverse = self.rope = None
        if self.span is None:
            return None
        start, stop, grid = self.span
        h, rope = args[0], args[3]
        if not (torch.is_tensor(h) and h.ndim == 2 and h.shape[0] >= stop):
            _log_once(f"hidden states do not cover the video span {(start, stop)}; inactive")
            return None
        if not (torch.is_tensor(rope) and rope.ndim >= 2 and rope.shape[1] == h.shape[0]):
            shape = tuple(rope.shape) if torch.is_tensor(rope) else type(rope).__name__
            _log_once(f"rope table {shape} does not match {h.shape[0]} tokens; inactive")
            return None
        forward, self.inverse = _composed(grid, self.curve, h.device, start, stop, h.shape[0],
                                          self.block)
        # The rotation table is elementwise per row, so permuting its rows is
        # permuting the positions.
        self.rope = _gather(rope, forward.to(rope.device), 1)
        return (_gather(h, forward, 0),) + tuple(args[1:3]) + (self.rope,) + tuple(args[4:])

    def after_stack(self, _module, _args, output):
        inverse, span = self.inverse, self.span
        self.inverse = self.rope = None
        if inverse is None or span is None:
            return None
        if not (torch.is_tensor(output) and output.shape[0] >= span[1]
                and output.shape[0] == inverse.numel()):
            shape = tuple(output.shape) if torch.is_tensor(output) else type(output).__name__
            logging.error(f"[sol_attn] H3 Morton: block stack changed the token count ({shape}); "
                          "cannot restore order")
            return None
        return _gather(output, inverse, 0)


def install_h3_morton(model, block=None):
    """Install the H3 hooks once per model (/root/reference/_morton_h3.py:110-226).
    Reordering is inert without transformer_options['sol_morton']; the video
    span is published for the conditioning sink on every pass."""
    if model in _H3Reorder.installed:
        return
    for attr in ("rope_freqs", "_forward", "blocks"):
        if not hasattr(model, attr):
            raise RuntimeError(f"MiniMax-H3 Morton needs .{attr} on the diffusion model")
    _SPANS.watch(sys.modules[type(model).__module__])
    state = _H3Reorder(model, BLOCK_SIZE if block is None else int(block))
    model._forward = state.wrap_forward(model._forward)
    model.rope_freqs = state.wrap_rope(model.rope_freqs)
    for blk in model.blocks:
        blk.register_forward_pre_hook(state.before_block)
    model.blocks[-1].register_forward_hook(state.after_stack)
    _H3Reorder.installed.add(model)


install_h3_hooks = install_h3_morton
