"""Composition with object-patched attention forwards.

A forward-level patch (an attention module's ``forward`` replaced, e.g. a
memory-efficient Sage patch) never reaches ``optimized_attention``, so there
is no override to chain onto. Instead the patched forward is wrapped: calls
Sol-Attn would take (self-attention on a bf16 GPU tensor of at least
``min_tokens`` tokens, inside the sigma window) run the module's stock forward
(which reaches the override), or a cooperating patch's ``sol_take_forward``;
every other call keeps the patch (/root/reference/__init__.py:345-419).

The gate parameters come from transformer_options['sol_compose'], which the
node publishes; without it the patch runs as it is.
"""

from __future__ import annotations

import weakref

import torch

from ._dispatch import _log_once


def _options_of(args, kwargs):
    options = kwargs.get("transformer_options")
    if isinstance(options, dict):
        return options
    for value in args:
        if isinstance(value, dict) and "sol_compose" in value:
            return value
    return {}


def _hidden_states(args):
    """(x as passed, the tensor inside it). A low-VRAM block patch passes x as a
    one-element list the forward is expected to empty."""
    x = args[0] if args else None
    if isinstance(x, list) and len(x) == 1 and torch.is_tensor(x[0]):
        return x, x[0]
    return x, x


def _sol_takes(gate, tensor, options) -> bool:
    if gate is None or not torch.is_tensor(tensor):
        return False
    if tensor.device.type != "cuda" or tensor.dtype != torch.bfloat16 or tensor.ndim not in (2, 3):
        return False
    # MiniMax-H3 packs tokens first (S, C); Wan-style models are batch-first.
    tokens = tensor.shape[0] if tensor.ndim == 2 else tensor.shape[1]
    if tokens < gate["min_tokens"]:
        return False
    sigmas = options.get("sigmas")
    if sigmas is None:
        return True
    sigma = float(sigmas[0])
    return gate["sigma_end"] <= sigma <= gate["sigma_start"]


class ComposedForward:
    """Replacement ``forward`` for an attention module whose forward was patched."""

    _sol_composed = True

    def __init__(self, module, patched_forward):
        self.module = module
        self.patched = patched_forward
        self.stock = type(module).forward

    def __call__(self, *args, **kwargs):
        options = _options_of(args, kwargs)
        x, tensor = _hidden_states(args)
        if not _sol_takes(options.get("sol_compose"), tensor, options):
            return self.patched(*args, **kwargs)
        delegate = options.get("sol_take_forward")
        if delegate is not None:
            return delegate(self.module, *args, **kwargs)
        if tensor is not x:  # consume the hand-off list, pass the tensor itself
            x.clear()
            args = (tensor,) + tuple(args[1:])
        return self.stock(self.module, *args, **kwargs)


def _compose_module_patch(module, patched_forward):
    return ComposedForward(module, patched_forward)


def _needs_composing(attn) -> bool:
    forward = attn.__dict__.get("forward")
    if forward is None or getattr(forward, "_sol_composed", False):
        return False
    if getattr(forward, "_uses_optimized_attention", False):
        return False  # it reaches optimized_attention itself; the override applies
    # an un-patch leaves the stock forward bound on the instance
    return getattr(forward, "__func__", None) is not type(attn).forward


class _ComposeHook:
    """Block pre-hook that wraps a foreign attention forward just before the
    block runs, so patches applied after the node (which overwrite the same
    object-patch key) still compose at sampling time."""

    hooked = weakref.WeakSet()  # models with the hooks

    def __init__(self, attn_attr):
        self.attn_attr = attn_attr

    def __call__(self, block, _args):
        attn = getattr(block, self.attn_attr, None)
        if attn is None or not _needs_composing(attn):
            return None
        attn.forward = ComposedForward(attn, attn.__dict__["forward"])
        _log_once(("composed", self.attn_attr),
                  f"composing with a patched {self.attn_attr}.forward; Sol-Attn takes eligible "
                  "self-attention calls, the patch keeps the rest")
        return None


def _install_compose_hooks(model, attn_attr):
    if model in _ComposeHook.hooked:
        return
    hook = _ComposeHook(attn_attr)
    for block in model.blocks:
        block.register_forward_pre_hook(hook)
    _ComposeHook.hooked.add(model)
