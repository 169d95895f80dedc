"""Attention-override dispatch: gates, layout adaptation, kernel choice, stats.

The ComfyUI-facing behaviour of /root/reference/__init__.py:43-342 without the
ComfyUI imports, so it can be exercised on its own:

* ``make_override`` builds the ``optimized_attention_override`` callable: mask
  -> dense; ``dense_blocks`` / ``tau_profile`` by the running block index; the
  sigma window; the MiniMax-H3 conditioning sink; then the kernel, with any
  exception counted, logged and answered with the dense path.
* ``_run`` adapts BHND or B,N,(H*D) inputs to BTHD views without copies, checks
  eligibility and calls the bf16 or int8 kernel.
* ``make_probe_override`` computes every call both ways and records the
  per-block relative error (the Block Probe).
"""

from __future__ import annotations

import logging
import re
from functools import partial

import torch

try:
    from ._tri_fwd import sol_attn as _sol_attn_kernel
    _IMPORT_ERROR = None
except Exception as exc:  # missing or unloadable libsolattn.so
    _sol_attn_kernel = None
    _IMPORT_ERROR = exc

try:
    from ._int8_fwd import sol_attn_int8 as _sol_attn_int8_kernel
    _INT8_IMPORT_ERROR = None
except Exception as exc:
    _sol_attn_int8_kernel = None
    _INT8_IMPORT_ERROR = exc

HEAD_DIM = 128
BLOCK_SIZE = 64  # default routing block (the reference's); 128 is also supported

_stats = {"sparse": 0, "dense_fallback": 0, "outside_range": 0, "dense_block": 0, "errors": 0}
_seen: set = set()
_BLOCK_INDEX_HOOKED: set = set()
_probe: dict = {}

_SPEC = re.compile(r"(-?\d+)(?:-(-?\d+))?")


def parse_blocks(spec, count):
    """"0-3,47,-1" -> frozenset of block indices in [0, count); negative indices
    count from the end, reversed ranges are swapped, whitespace is ignored
    (/root/reference/__init__.py:49-66)."""
    picked = set()
    for part in re.sub(r"\s+", "", str(spec)).split(","):
        if not part:
            continue
        m = _SPEC.fullmatch(part)
        if m is None:
            raise ValueError(f"cannot parse block spec {part!r}; use indices and ranges like '0-3,47,-1'")
        lo = int(m.group(1))
        hi = lo if m.group(2) is None else int(m.group(2))
        lo, hi = (x + count if x < 0 else x for x in (lo, hi))
        lo, hi = min(lo, hi), max(lo, hi)
        picked.update(range(max(lo, 0), min(hi, count - 1) + 1))
    return frozenset(picked)


def parse_tau_profile(spec, count):
    """"0-30=2.0; 39-42=0.9" -> {block: tau}. Entries split on ';' or newlines,
    '#' starts a comment, later entries win (/root/reference/__init__.py:69-91)."""
    profile = {}
    for raw in re.split(r"[;\n]", str(spec)):
        entry = raw.split("#", 1)[0].strip()
        if not entry:
            continue
        blocks, sep, value = entry.partition("=")
        if not sep:
            raise ValueError(f"tau_profile entry {entry!r} needs '=', e.g. '39-42=0.9'")
        try:
            level = float(value)
        except ValueError:
            raise ValueError(f"tau_profile entry {entry!r} has a non-numeric tau") from None
        profile.update(dict.fromkeys(parse_blocks(blocks, count), level))
    return profile


def _install_block_index(model):
    """Publish the running block index as transformer_options['sol_block']
    (/root/reference/__init__.py:94-113). False if the model has no .blocks."""
    blocks = getattr(model, "blocks", None)
    if blocks is None:
        return False
    if id(model) in _BLOCK_INDEX_HOOKED:
        return True

    def publisher(index):
        def hook(_module, _args, kwargs):
            options = kwargs.get("transformer_options")
            if isinstance(options, dict):
                options["sol_block"] = index
        return hook

    for index, block in enumerate(blocks):
        block.register_forward_pre_hook(publisher(index), with_kwargs=True)
    _BLOCK_INDEX_HOOKED.add(id(model))
    return True


def _probe_record(block, sparse_out, reference):
    """Accumulate this block's ||sparse - dense|| / ||dense||."""
    ref = reference.float()
    norm = ref.norm()
    if norm > 0:
        total, calls = _probe.get(block, (0.0, 0))
        _probe[block] = (total + float((sparse_out.float() - ref).norm() / norm), calls + 1)


def log_probe_summary(*_args, **_kwargs):
    """Per-block sensitivity, worst first (/root/reference/__init__.py:129-141)."""
    if not _probe:
        return
    rows = sorted(((total / calls, block, calls) for block, (total, calls) in _probe.items()),
                  key=lambda r: (r[0], -1 if r[1] is None else r[1]), reverse=True)
    logging.info("[sol_attn] block sensitivity to sparsification (worst first); "
                 "put the top entries in dense_blocks:")
    for error, block, calls in rows:
        label = f"{block:3d}" if isinstance(block, int) else str(block)
        logging.info(f"[sol_attn]   block {label}  rel err {error:.4f}  ({calls} calls)")
    _probe.clear()


def sol_attn_stats():
    """Dispatch counters since process start (or the last reset)."""
    return dict(_stats)


def reset_sol_attn_stats():
    for key in _stats:
        _stats[key] = 0
    _seen.clear()


def _log_once(key, message):
    if key not in _seen:
        _seen.add(key)
        logging.info(f"[sol_attn] {message}")


def _log_kernel_failure(exc):
    # Full traceback the first time a distinct failure is seen, one line after.
    key = ("kernel_failure", type(exc).__name__, str(exc))
    first = key not in _seen
    _seen.add(key)
    logging.error(f"[sol_attn] kernel failed ({exc}); falling back", exc_info=first)


def _ineligible(q, k, mask, dim_head, min_tokens):
    """Why this call cannot take the sparse kernel, or None
    (/root/reference/__init__.py:170-189). q/k are BTHD."""
    if _sol_attn_kernel is None:
        return f"kernel import failed: {_IMPORT_ERROR}"
    if q.device.type != "cuda":
        return "not cuda"
    if q.dtype != torch.bfloat16:
        return f"dtype {q.dtype} (kernel is bf16-only)"
    if dim_head != HEAD_DIM:
        return f"head_dim {dim_head} != {HEAD_DIM}"
    if mask is not None:
        return "masked attention"
    if q.shape[1] != k.shape[1]:
        return "cross-attention (kept dense)"
    if q.shape != k.shape:
        return f"q/k shape mismatch {tuple(q.shape)} vs {tuple(k.shape)}"
    if q.shape[1] < min_tokens:
        return f"seq {q.shape[1]} < {min_tokens}"
    return None


def _run(q, k, v, heads, skip_reshape, skip_output_reshape, scale, tau, min_tokens, verbose,
         int8_qk=False, sink_blocks=(0, 0), sink_q=(0, 0), use_tma=False, int8_pv=True,
         block=BLOCK_SIZE):
    """The attention output, or None if this call stays dense
    (/root/reference/__init__.py:192-231)."""
    if skip_reshape:  # BHND
        b, _, _, dim_head = q.shape
        qs, ks, vs = (t.transpose(1, 2) for t in (q, k, v))
    else:  # B, N, heads * dim_head
        b, _, width = q.shape
        dim_head = width // heads
        qs, ks, vs = (t.view(b, -1, heads, dim_head) for t in (q, k, v))

    reason = _ineligible(qs, ks, None, dim_head, min_tokens)
    if reason is not None:
        _stats["dense_fallback"] += 1
        if verbose:
            _log_once((tuple(qs.shape), reason), f"dense {tuple(qs.shape)}: {reason}")
        return None

    # Strided views go straight to the kernels (no contiguous() here).
    if int8_qk:
        if _sol_attn_int8_kernel is None:
            raise RuntimeError(f"Sol-Attn INT8 kernel unavailable: {_INT8_IMPORT_ERROR}")
        out = _sol_attn_int8_kernel(qs, ks, vs, scale=scale, tau=tau, sink_blocks=sink_blocks,
                                    sink_q=sink_q, use_tma=use_tma, int8_pv=int8_pv, block=block)
    else:
        out = _sol_attn_kernel(qs, ks, vs, scale=scale, tau=tau, sink_blocks=sink_blocks,
                               sink_q=sink_q, use_tma=use_tma, block=block)
    _stats["sparse"] += 1
    if verbose:
        mode = "int8" if int8_qk else "bf16"
        _log_once((tuple(qs.shape), "sparse", mode, block),
                  f"sparse {tuple(qs.shape)} tau={tau} {mode} block={block} hip")
    if skip_output_reshape:
        return out.transpose(1, 2)  # BHND
    return out.reshape(b, -1, heads * dim_head)


def _sink_blocks(transformer_options, tokens, mode, block=BLOCK_SIZE):
    """(exact-KV blocks, dense-query blocks) covering MiniMax-H3's packed
    conditioning rows before the video span (/root/reference/__init__.py:237-253)."""
    if mode == "off":
        return (0, 0), (0, 0)
    span = (transformer_options or {}).get("sol_h3_video_span")
    if span is None:
        return (0, 0), (0, 0)
    video_start, video_stop = span
    if tokens < video_stop or video_start <= 0:
        return (0, 0), (0, 0)
    kv = (0, -(-int(video_start) // int(block)))
    return kv, (kv if mode == "exact_kv_and_rows" else (0, 0))


def make_override(tau=1.0, min_tokens=4096, sigma_start=None, sigma_end=None, verbose=False,
                  int8_qk=False, sink_conditioning="exact_kv", use_tma=False,
                  dense_blocks=frozenset(), tau_profile=None, int8_pv=True, previous=None,
                  block=BLOCK_SIZE):
    """An optimized_attention_override callable (/root/reference/__init__.py:256-320).
    ``previous`` (an override already on the model) gets every call this one
    declines before ``func`` does."""

    def override(func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                 skip_output_reshape=False, **kwargs):
        def dense():
            target = func if previous is None else partial(previous, func)
            return target(q, k, v, heads, mask=mask, attn_precision=attn_precision,
                          skip_reshape=skip_reshape, skip_output_reshape=skip_output_reshape,
                          **kwargs)

        if mask is not None:
            _stats["dense_fallback"] += 1
            return dense()

        options = kwargs.get("transformer_options", {})
        index = options.get("sol_block") if (dense_blocks or tau_profile) else None
        if index in dense_blocks:
            _stats["dense_block"] += 1
            return dense()
        level = tau_profile.get(index, tau) if tau_profile else tau

        # Sampling window: dense outside [sigma_end, sigma_start] (warm-up steps).
        if sigma_start is not None or sigma_end is not None:
            sigmas = options.get("sigmas")
            if sigmas is not None:
                sigma = float(sigmas[0])
                if (sigma_start is not None and sigma > sigma_start) or \
                        (sigma_end is not None and sigma < sigma_end):
                    _stats["outside_range"] += 1
                    return dense()

        tokens = q.shape[2] if skip_reshape else q.shape[1]
        sink, sink_q = _sink_blocks(options, tokens, sink_conditioning, block)
        if verbose and sink != (0, 0):
            _log_once((tokens, sink, sink_q),
                      f"conditioning sink: KV blocks {sink} exact, dense query blocks {sink_q}")
        try:
            out = _run(q, k, v, heads, skip_reshape, skip_output_reshape, kwargs.get("scale"),
                       level, min_tokens, verbose, int8_qk, sink, sink_q, use_tma, int8_pv, block)
        except Exception as exc:
            _stats["errors"] += 1
            _log_kernel_failure(exc)
            return dense()
        return dense() if out is None else out

    return override


def make_probe_override(inner):
    """Run every call sparse and dense, record the per-block error, return the
    dense result so each block is measured on a clean input
    (/root/reference/__init__.py:323-342)."""

    def override(func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                 skip_output_reshape=False, **kwargs):
        common = dict(mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
                      skip_output_reshape=skip_output_reshape, **kwargs)
        sparse = inner(func, q, k, v, heads, **common)
        reference = func(q, k, v, heads, **common)
        _probe_record(kwargs.get("transformer_options", {}).get("sol_block"), sparse, reference)
        return reference

    return override


def _compose_module_patch(module, patched_forward):
    """Gate an object-patched attention forward: calls Sol-Attn would take run
    the stock forward (and so reach the override); the rest keep the patch.
    Gate parameters come from transformer_options['sol_compose']
    (/root/reference/__init__.py:345-385)."""
    stock = type(module).forward

    def forward(*args, **kwargs):
        options = kwargs.get("transformer_options")
        if not isinstance(options, dict):
            options = next((a for a in args if isinstance(a, dict) and "sol_compose" in a), {})
        gate = options.get("sol_compose")
        x = args[0] if args else None
        # A low-VRAM block patch hands x over in a one-item list.
        tensor = x[0] if isinstance(x, list) and len(x) == 1 and torch.is_tensor(x[0]) else x
        take = (gate is not None and torch.is_tensor(tensor) and tensor.device.type == "cuda"
                and tensor.dtype == torch.bfloat16 and tensor.ndim in (2, 3))
        if take:
            tokens = tensor.shape[0] if tensor.ndim == 2 else tensor.shape[1]
            take = tokens >= gate["min_tokens"]
        if take:
            sigmas = options.get("sigmas")
            if sigmas is not None:
                sigma = float(sigmas[0])
                take = not (sigma > gate["sigma_start"] or sigma < gate["sigma_end"])
        if take:
            delegate = options.get("sol_take_forward")
            if delegate is not None:
                return delegate(module, *args, **kwargs)
            if tensor is not x:
                x.clear()
                args = (tensor,) + args[1:]
            return stock(module, *args, **kwargs)
        return patched_forward(*args, **kwargs)

    forward._sol_composed = True
    return forward


_COMPOSE_HOOKED: set = set()


def _install_compose_hooks(model, attn_attr):
    """Re-wrap any foreign attention forward before each block runs, so patches
    applied after the node still compose (/root/reference/__init__.py:391-419)."""
    if id(model) in _COMPOSE_HOOKED:
        return

    def pre_hook(block, _args):
        attn = getattr(block, attn_attr, None)
        if attn is None:
            return None
        fwd = attn.__dict__.get("forward")
        if fwd is None or getattr(fwd, "_sol_composed", False):
            return None
        if getattr(fwd, "_uses_optimized_attention", False):
            return None
        if getattr(fwd, "__func__", None) is type(attn).forward:
            return None
        attn.forward = _compose_module_patch(attn, fwd)
        _log_once(("composed", attn_attr),
                  f"composing with a patched {attn_attr}.forward; Sol-Attn takes eligible "
                  "self-attention calls, the patch keeps the rest")
        return None

    for block in model.blocks:
        block.register_forward_pre_hook(pre_hook)
    _COMPOSE_HOOKED.add(id(model))
