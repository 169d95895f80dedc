"""The Block Probe's measurement: every attention call computed sparse and
dense, the relative error accumulated per transformer block
(/root/reference/__init__.py:116-141, 323-342).

The probe answers with the dense result, so each block is measured on the
input a dense run would give it: returning the sparse result would let early
error compound into every later block's number.
"""

from __future__ import annotations

import logging

# block index (or None when the model publishes none) -> (sum of rel. errors, calls)
_probe: dict = {}


def _probe_record(block, sparse_out, reference):
    """Add ||sparse - dense|| / ||dense|| for one call of ``block``."""
    dense = reference.float()
    scale = dense.norm()
    if scale > 0:
        error = float((sparse_out.float() - dense).norm() / scale)
        total, calls = _probe.get(block, (0.0, 0))
        _probe[block] = (total + error, calls + 1)


def _ranked():
    """(mean error, block, calls), worst first; unnamed blocks sort last among equals."""
    rows = [(total / calls, block, calls) for block, (total, calls) in _probe.items()]
    return sorted(rows, key=lambda r: (r[0], -1 if r[1] is None else r[1]), reverse=True)


def log_probe_summary(*_args, **_kwargs):
    """Log the per-block sensitivity worst first and clear the record (the
    node registers this as the model's cleanup callback)."""
    if not _probe:
        return
    logging.info("[sol_attn] block sensitivity to sparsification (worst first); "
                 "put the top entries in dense_blocks:")
    for error, block, calls in _ranked():
        label = f"{block:3d}" if isinstance(block, int) else str(block)
        logging.info(f"[sol_attn]   block {label}  rel err {error:.4f}  ({calls} calls)")
    _probe.clear()


class ProbeOverride:
    """Wraps an installed override: runs it (sparse) and ``func`` (dense) on
    every call, records the error under transformer_options['sol_block'] and
    returns the dense output."""

    def __init__(self, inner):
        self.inner = inner

    def __call__(self, func, q, k, v, heads, mask=None, attn_precision=None,
                 skip_reshape=False, skip_output_reshape=False, **kwargs):
        same = dict(mask=mask, attn_precision=attn_precision, skip_reshape=skip_reshape,
                    skip_output_reshape=skip_output_reshape, **kwargs)
        sparse = self.inner(func, q, k, v, heads, **same)
        dense = func(q, k, v, heads, **same)
        block = (kwargs.get("transformer_options") or {}).get("sol_block")
        _probe_record(block, sparse, dense)
        return dense


def make_probe_override(inner):
    return ProbeOverride(inner)
