"""Attention-override dispatch: which calls take the sparse kernels, and how.

The ComfyUI-facing behaviour of /root/reference/__init__.py:43-320, organised
around three objects instead of closures:

* ``SparsePolicy``: the node's settings for one patched model (tau, the
  sigma window, depth controls, INT8 switches, sink mode, block size).
* ``AttentionCall``: one call of the override protocol with its layout
  normalised (BTHD views of q/k/v, the transformer options, token count) and
  a ``restore`` that maps a BTHD result back to the caller's layout.
* ``SolAttnOverride``: the ``optimized_attention_override`` callable. It walks
  an ordered gate table (mask, dense block, sigma window); the first gate that
  refuses names the ``_stats`` counter to bump and the call goes dense (to the
  previous override if one was chained, else ``func``). Calls that pass get the
  H3 conditioning sink, the eligibility checks and the kernel; any exception is
  counted, logged once with its traceback and answered densely.

The gate order, ``_stats`` keys, eligibility reasons, block/tau-profile syntax
and the sink rule are the reference's (they are the drop-in boundary); the
structure is this module's own.
"""

from __future__ import annotations

import logging
import weakref
from dataclasses import dataclass, field
from typing import Callable, Optional

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
# Shortest sequence the sparse path takes by default: the reference's 4096
# (/root/reference/__init__.py:256, 442, 657), so calls of 2048-4095 tokens stay
# exact (dense) as there. On MI355X every sparse call (BF16 and both INT8
# modes, prep included) already beats dense PyTorch SDPA from 2048 tokens, so
# a node may lower its min_tokens to 2048 to trade that exactness for speed.
MIN_TOKENS = 4096
BLOCK_SIZE = 64  # default routing block (the reference's); 128 is also supported
# Query/key blocks per head the forward kernels take; longer sequences stay dense.
MAX_BLOCKS = 16384

STAT_KEYS = ("sparse", "dense_fallback", "outside_range", "dense_block", "errors")
_stats = dict.fromkeys(STAT_KEYS, 0)
_seen: set = set()


# ------------------------------------------------------------------ logging
def _log_once(key, message):
    if key in _seen:
        return
    _seen.add(key)
    logging.info(f"[sol_attn] {message}")


def _log_kernel_failure(exc):
    """ERROR line per failure; the traceback only the first time a given
    failure (type and message) is seen, so a failing run stays readable."""
    key = ("kernel_failure", type(exc).__name__, str(exc))
    first_time = key not in _seen
    _seen.add(key)
    logging.error(f"[sol_attn] kernel failed ({exc}); falling back", exc_info=first_time)


def sol_attn_stats():
    """Dispatch counters since process start (or the last reset)."""
    return dict(_stats)


def reset_sol_attn_stats():
    _stats.update(dict.fromkeys(STAT_KEYS, 0))
    _seen.clear()


# --------------------------------------------------------- block selection
def _parse_index(text: str, whole: str) -> int:
    body = text[1:] if text.startswith("-") else text
    if not body.isdigit():
        raise ValueError(f"cannot parse block spec {whole!r}; use indices and ranges like '0-3,47,-1'")
    return int(text)


def _split_range(part: str):
    """'5' -> (5, 5); '2-7' -> (2, 7); '-3--1' -> (-3, -1). The separator is the
    first '-' that follows a digit."""
    for pos in range(1, len(part)):
        if part[pos] == "-" and part[pos - 1].isdigit():
            return _parse_index(part[:pos], part), _parse_index(part[pos + 1:], part)
    value = _parse_index(part, part)
    return value, value


def parse_blocks(spec, count):
    """Block indices named by ``spec`` ("0-3,47,-1"), as a frozenset within
    [0, count). Whitespace anywhere is ignored, negative indices count from the
    end, a reversed range is read forwards, and indices outside the model are
    dropped (/root/reference/__init__.py:49-66)."""
    chosen = set()
    compact = "".join(str(spec).split())
    for part in filter(None, compact.split(",")):
        first, last = (i + count if i < 0 else i for i in _split_range(part))
        if first > last:
            first, last = last, first
        chosen.update(range(max(first, 0), min(last, count - 1) + 1))
    return frozenset(chosen)


def parse_tau_profile(spec, count):
    """{block: tau} from "0-30=2.0; 39-42=0.9". Entries are separated by ';' or
    newlines, '#' starts a comment, the block side takes ``parse_blocks``
    syntax and later entries override earlier ones
    (/root/reference/__init__.py:69-91)."""
    profile = {}
    for line in str(spec).replace(";", "\n").split("\n"):
        entry = line.partition("#")[0].strip()
        if not entry:
            continue
        if "=" not in entry:
            raise ValueError(f"tau_profile entry {entry!r} needs '=', e.g. '39-42=0.9'")
        blocks, _, value = entry.partition("=")
        try:
            level = float(value)
        except ValueError:
            raise ValueError(f"tau_profile entry {entry!r} has a non-numeric tau") from None
        for index in parse_blocks(blocks, count):
            profile[index] = level
    return profile


class _BlockIndexPublisher:
    """One forward pre-hook per block that writes the block's position into
    transformer_options['sol_block'] (/root/reference/__init__.py:94-113)."""

    installed = weakref.WeakSet()  # models with the hooks

    def __init__(self, blocks):
        self.position = {id(block): index for index, block in enumerate(blocks)}

    def __call__(self, module, _args, kwargs):
        options = kwargs.get("transformer_options")
        if isinstance(options, dict):
            options["sol_block"] = self.position[id(module)]


def _install_block_index(model):
    """Publish the running block index; False when the model has no .blocks."""
    blocks = getattr(model, "blocks", None)
    if blocks is None:
        return False
    if model not in _BlockIndexPublisher.installed:
        publisher = _BlockIndexPublisher(blocks)
        for block in blocks:
            block.register_forward_pre_hook(publisher, with_kwargs=True)
        _BlockIndexPublisher.installed.add(model)
    return True


# ------------------------------------------------------------ the call site
@dataclass
class AttentionCall:
    """One call of the override protocol, normalised to BTHD views."""

    q: torch.Tensor
    k: torch.Tensor
    v: torch.Tensor
    heads: int
    mask: Optional[torch.Tensor]
    skip_reshape: bool
    skip_output_reshape: bool
    kwargs: dict

    @property
    def options(self) -> dict:
        return self.kwargs.get("transformer_options") or {}

    @property
    def tokens(self) -> int:
        return self.q.shape[2] if self.skip_reshape else self.q.shape[1]

    def bthd(self):
        """(q, k, v, dim_head) as BTHD views; no data is copied. Input layouts:
        BHND when skip_reshape, else [B, N, heads*dim_head]."""
        if self.skip_reshape:
            return (*(t.transpose(1, 2) for t in (self.q, self.k, self.v)), self.q.shape[-1])
        batch, _, width = self.q.shape
        dim_head = width // self.heads
        return (*(t.view(batch, -1, self.heads, dim_head) for t in (self.q, self.k, self.v)),
                dim_head)

    def restore(self, out: torch.Tensor) -> torch.Tensor:
        """A BTHD result in the layout the caller expects."""
        if self.skip_output_reshape:
            return out.transpose(1, 2)
        return out.reshape(out.shape[0], -1, out.shape[2] * out.shape[3])


# Eligibility, checked in this order; each entry gives the reason text when
# the call cannot take the kernel (/root/reference/__init__.py:170-189).
def _eligibility_checks(q, k, mask, dim_head, min_tokens, block):
    yield _sol_attn_kernel is None, lambda: f"kernel import failed: {_IMPORT_ERROR}"
    yield q.device.type != "cuda", lambda: "not cuda"
    yield q.dtype != torch.bfloat16, lambda: f"dtype {q.dtype} (kernel is bf16-only)"
    yield dim_head != HEAD_DIM, lambda: f"head_dim {dim_head} != {HEAD_DIM}"
    yield mask is not None, lambda: "masked attention"
    yield q.shape[1] != k.shape[1], lambda: "cross-attention (kept dense)"
    yield q.shape != k.shape, lambda: f"q/k shape mismatch {tuple(q.shape)} vs {tuple(k.shape)}"
    yield q.shape[1] < min_tokens, lambda: f"seq {q.shape[1]} < {min_tokens}"
    blocks = -(-q.shape[1] // block)
    yield blocks > MAX_BLOCKS, lambda: (f"seq {q.shape[1]} makes {blocks} blocks of {block}, "
                                        f"more than the kernels' {MAX_BLOCKS}")


def _ineligible(q, k, mask, dim_head, min_tokens, block=BLOCK_SIZE):
    """Why this call cannot take the sparse kernel, or None. q/k are BTHD."""
    for refused, reason in _eligibility_checks(q, k, mask, dim_head, min_tokens, block):
        if refused:
            return reason()
    return None


def _run(q, k, v, heads, skip_reshape, skip_output_reshape, scale, tau, min_tokens, verbose,
         int8_qk=False, sink_blocks=(0, 0), sink_q=(0, 0), use_tma=False, int8_pv=True,
         block=BLOCK_SIZE, pv_codes="block"):
    """The sparse attention output in the caller's layout, or None when the
    call stays dense (/root/reference/__init__.py:192-231). Strided views go
    to the kernels as they are."""
    call = AttentionCall(q, k, v, heads, None, skip_reshape, skip_output_reshape, {})
    qs, ks, vs, dim_head = call.bthd()
    reason = _ineligible(qs, ks, None, dim_head, min_tokens, block)
    if reason is not None:
        _stats["dense_fallback"] += 1
        if verbose:
            _log_once((tuple(qs.shape), reason), f"dense {tuple(qs.shape)}: {reason}")
        return None
    args = dict(scale=scale, tau=tau, sink_blocks=sink_blocks, sink_q=sink_q, use_tma=use_tma,
                block=block)
    if int8_qk:
        if _sol_attn_int8_kernel is None:
            raise RuntimeError(f"Sol-Attn INT8 kernel unavailable: {_INT8_IMPORT_ERROR}")
        out = _sol_attn_int8_kernel(qs, ks, vs, int8_pv=int8_pv, pv_codes=pv_codes, **args)
    else:
        out = _sol_attn_kernel(qs, ks, vs, **args)
    _stats["sparse"] += 1
    if verbose:
        mode = "int8" if int8_qk else "bf16"
        _log_once((tuple(qs.shape), "sparse", mode, block),
                  f"sparse {tuple(qs.shape)} tau={tau} {mode} block={block} hip")
    return call.restore(out)


def _sink_blocks(transformer_options, tokens, mode, block=BLOCK_SIZE):
    """(exact-KV block range, dense-query block range) that cover MiniMax-H3's
    packed conditioning rows, i.e. every block holding a row before the video
    span (/root/reference/__init__.py:237-253)."""
    none = ((0, 0), (0, 0))
    span = (transformer_options or {}).get("sol_h3_video_span")
    if mode == "off" or span is None:
        return none
    video_start, video_stop = span
    if video_start <= 0 or tokens < video_stop:
        return none
    covering = (0, -(-int(video_start) // int(block)))
    return covering, covering if mode == "exact_kv_and_rows" else (0, 0)


# --------------------------------------------------------------- the policy
@dataclass(frozen=True)
class SparsePolicy:
    """What the Patch Sol-Attn node configured for one model."""

    tau: float = 1.0
    min_tokens: int = MIN_TOKENS
    sigma_start: Optional[float] = None
    sigma_end: Optional[float] = None
    verbose: bool = False
    int8_qk: bool = False
    sink_conditioning: str = "exact_kv"
    use_tma: bool = False
    dense_blocks: frozenset = frozenset()
    tau_profile: Optional[dict] = field(default=None, hash=False)
    int8_pv: bool = True
    block: int = BLOCK_SIZE
    pv_codes: str = "block"  # int8 P codes: against each block's max, or "running"

    def block_index(self, call: AttentionCall):
        if not (self.dense_blocks or self.tau_profile):
            return None
        return call.options.get("sol_block")

    def tau_for(self, index) -> float:
        return self.tau_profile.get(index, self.tau) if self.tau_profile else self.tau

    def outside_window(self, call: AttentionCall) -> bool:
        """The paper's dense warm-up: sigma above sigma_start or below sigma_end."""
        if self.sigma_start is None and self.sigma_end is None:
            return False
        sigmas = call.options.get("sigmas")
        if sigmas is None:
            return False
        sigma = float(sigmas[0])
        return ((self.sigma_start is not None and sigma > self.sigma_start)
                or (self.sigma_end is not None and sigma < self.sigma_end))


# Gates in the reference's order: (stats key, refuses?).
_GATES: tuple = (
    ("dense_fallback", lambda policy, call: call.mask is not None),
    ("dense_block", lambda policy, call: policy.block_index(call) in policy.dense_blocks),
    ("outside_range", lambda policy, call: policy.outside_window(call)),
)


class SolAttnOverride:
    """The ``optimized_attention_override`` callable for one policy.

    ``previous`` (an override already on the model) gets every call this one
    declines before ``func`` does."""

    def __init__(self, policy: SparsePolicy, previous: Optional[Callable] = None):
        self.policy = policy
        self.previous = previous

    def dense(self, func, call: AttentionCall, attn_precision):
        target = func if self.previous is None else (
            lambda *a, **kw: self.previous(func, *a, **kw))
        return target(call.q, call.k, call.v, call.heads, mask=call.mask,
                      attn_precision=attn_precision, skip_reshape=call.skip_reshape,
                      skip_output_reshape=call.skip_output_reshape, **call.kwargs)

    def __call__(self, func, q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                 skip_output_reshape=False, **kwargs):
        policy = self.policy
        call = AttentionCall(q, k, v, heads, mask, skip_reshape, skip_output_reshape, kwargs)
        for counter, refuses in _GATES:
            if refuses(policy, call):
                _stats[counter] += 1
                return self.dense(func, call, attn_precision)
        tau = policy.tau_for(policy.block_index(call))
        sink, sink_q = _sink_blocks(call.options, call.tokens, policy.sink_conditioning,
                                    policy.block)
        if policy.verbose and sink != (0, 0):
            _log_once((call.tokens, sink, sink_q),
                      f"conditioning sink: KV blocks {sink} exact, dense query blocks {sink_q}")
        try:
            out = _run(q, k, v, heads, skip_reshape, skip_output_reshape, kwargs.get("scale"),
                       tau, policy.min_tokens, policy.verbose, policy.int8_qk, sink, sink_q,
                       policy.use_tma, policy.int8_pv, policy.block, policy.pv_codes)
        except Exception as exc:
            _stats["errors"] += 1
            _log_kernel_failure(exc)
            out = None
        return self.dense(func, call, attn_precision) if out is None else out


def make_override(tau=1.0, min_tokens=MIN_TOKENS, sigma_start=None, sigma_end=None, verbose=False,
                  int8_qk=False, sink_conditioning="exact_kv", use_tma=False,
                  dense_blocks=frozenset(), tau_profile=None, int8_pv=True, previous=None,
                  block=BLOCK_SIZE, pv_codes="block"):
    """An optimized_attention_override (/root/reference/__init__.py:256-320).
    ``pv_codes="running"`` (with int8_qk and int8_pv): P codes against the row's
    running max, an option of this build (the default is the reference's)."""
    policy = SparsePolicy(tau=tau, min_tokens=min_tokens, sigma_start=sigma_start,
                          sigma_end=sigma_end, verbose=verbose, int8_qk=int8_qk,
                          sink_conditioning=sink_conditioning, use_tma=use_tma,
                          dense_blocks=frozenset(dense_blocks), tau_profile=tau_profile or None,
                          int8_pv=int8_pv, block=int(block), pv_codes=pv_codes)
    return SolAttnOverride(policy, previous)


# The registry entry's policy: tau 1.0, MIN_TOKENS, BF16, no window, no sink
# (/root/reference/__init__.py:649-663).
REGISTRY_POLICY = SparsePolicy()


def try_sparse_default(q, k, v, heads, mask, skip_reshape, skip_output_reshape, scale):
    """The sparse output under REGISTRY_POLICY, or None (masked, ineligible, or
    the kernel failed; a failure is counted and logged)."""
    if mask is not None:
        return None
    policy = REGISTRY_POLICY
    try:
        return _run(q, k, v, heads, skip_reshape, skip_output_reshape, scale, policy.tau,
                    policy.min_tokens, False)
    except Exception as exc:
        _stats["errors"] += 1
        _log_kernel_failure(exc)
        return None


from ._probe import (  # noqa: E402,F401  (re-exported: the probe uses this module's stats)
    _probe,
    _probe_record,
    log_probe_summary,
    make_probe_override,
)
from ._compose import _compose_module_patch, _install_compose_hooks  # noqa: E402,F401
