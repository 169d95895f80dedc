"""Minimal stand-in for ComfyUI's comfy.ldm.modules.attention, for tests only."""

import torch

REGISTERED = {}


def attention_pytorch(q, k, v, heads, mask=None, attn_precision=None, skip_reshape=False,
                      skip_output_reshape=False, **kwargs):
    """Dense SDPA with ComfyUI's layout conventions (B,N,H*D or BHND)."""
    if skip_reshape:
        b, _, _, dim_head = q.shape
        qh, kh, vh = q, k, v
    else:
        b, _, width = q.shape
        dim_head = width // heads
        qh, kh, vh = (t.view(b, -1, heads, dim_head).transpose(1, 2) for t in (q, k, v))
    scale = kwargs.get("scale")
    out = torch.nn.functional.scaled_dot_product_attention(
        qh.float(), kh.float(), vh.float(), attn_mask=mask, scale=scale).to(q.dtype)
    if skip_output_reshape:
        return out
    return out.transpose(1, 2).reshape(b, -1, heads * dim_head)


def register_attention_function(name, fn):
    REGISTERED[name] = fn


def wrap_attn(fn):
    return fn


optimized_attention = attention_pytorch
optimized_attention_masked = attention_pytorch
