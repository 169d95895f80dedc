"""ctypes binding to libsolattn.so, the gfx950 HIP library (include/solattn.h).

The library is loaded at import; if it is missing or fails to load, importing
this module raises ImportError, so the kernel modules fail loudly (the node
layer records the error exactly as the reference records a Triton import
failure, /root/reference/__init__.py:25-38). There is no CPU fallback.
"""

from __future__ import annotations

import ctypes
import os

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("SOLATTN_LIB", os.path.join(_HERE, "libsolattn.so"))

_p = ctypes.c_void_p
_i = ctypes.c_int
_l = ctypes.c_int64
_f = ctypes.c_float

# Every exported symbol of include/solattn.h with its argument types.
SIGNATURES = {
    "solattn_last_error": ([], ctypes.c_char_p),
    "solattn_abi_version": ([], _i),
    "solattn_morton_perm": ([_l, _l, _l, _i, _l, _p, _p], _i),
    "solattn_reorder_rows": ([_p, _l, _l, _l, _p, _l, _l, _l, _l, _l, _p, _p], _i),
    "solattn_pool": ([_p, _l, _l, _l] * 3 + [_l] * 5 + [_p, _p, _l, _p, _p, _p], _i),
    "solattn_moments": ([_p, _l, _l, _l, _l, _l, _i, _p, _p, _p, _p, _p], _i),
    "solattn_route": ([_p, _p, _l, _p, _p, _l, _l, _l, _l, _l, _f, _f, _i, _l, _l, _l, _l,
                       _p, _p, _p, _p], _i),
    "solattn_quant_rows": ([_p, _l, _l, _l, _l, _l, _l, _l, _p, _p, _p, _l, _p], _i),
    "solattn_quant_rows_blocked": ([_p, _l, _l, _l, _l, _l, _l, _l, _p, _p, _p, _l, _p], _i),
    "solattn_quant_v": ([_p, _l, _l, _l, _l, _l, _l, _l, _p, _p, _l, _p], _i),
    "solattn_fwd_bf16": ([_p, _l, _l, _l] * 3 + [_p, _p, _l, _p, _p] + [_l] * 5 +
                         [_f, _p, _l, _l, _l, _p], _i),
    "solattn_fwd_int8": ([_p, _l, _l, _l, _p, _p, _p, _p, _p, _p, _p, _l, _l, _l, _l, _p, _p, _l,
                          _p, _p] + [_l] * 5 + [_f, _i, _p, _l, _l, _l, _p], _i),
    "solattn_prep_int8_sync_bytes": ([_l, _l], _l),
    "solattn_prep_int8": ([_p, _l, _l, _l] * 3 + [_l] * 5 + [_p, _p, _l] + [_p] * 9 + [_i, _p, _l,
                                                                              _p, _l, _p], _i),
    "solattn_sol_attn_workspace_bytes": ([_l, _l, _l, _l, _l, _i], _l),
    "solattn_sol_attn": ([_p, _l, _l, _l] * 3 + [_l] * 5 + [_f, _f, _l, _l, _l, _l, _p, _l,
                                                           _p, _l, _l, _l, _p], _i),
    "solattn_sol_attn_int8": ([_p, _l, _l, _l] * 3 + [_l] * 5 + [_f, _f, _l, _l, _l, _l, _i, _p,
                                                                _l, _p, _l, _l, _l, _p], _i),
    "solattn_sol_attn_int8_qblock": ([_p, _l, _l, _l] * 3 + [_l] * 5 + [_f, _f, _l, _l, _l, _l, _i,
                                                                       _p, _l, _p, _l, _l, _l, _p], _i),
    "solattn_sol_attn_noalloc": ([_p, _l, _l, _l] * 3 + [_l] * 5 + [_f, _f, _l, _l, _l, _l,
                                                                   _p, _l, _l, _l, _p], _i),
}

# Size of the per-device scratch array behind solattn_sol_attn_noalloc
# (SOLATTN_NOALLOC_SCRATCH_BYTES).
NOALLOC_SCRATCH_BYTES = 32 << 20
QUANT_BLOCK = 128  # tokens per scale of the per-block INT8 variant (SOLATTN_QUANT_BLOCK)


def _load() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libsolattn.so not found at {LIB_PATH}; build it with "
            f"`python {os.path.join(_HERE, 'build.py')}` (hipcc, gfx950)")
    try:
        lib = ctypes.CDLL(LIB_PATH)
    except OSError as exc:
        raise ImportError(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (args, res) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = args
        fn.restype = res
    return lib


LIB = _load()


class SolAttnError(RuntimeError):
    """A libsolattn call returned a nonzero status."""


def call(name: str, *args) -> None:
    """Call an entry point; raise SolAttnError with the library's message on failure."""
    rc = getattr(LIB, name)(*args)
    if rc != 0:
        msg = LIB.solattn_last_error().decode(errors="replace")
        raise SolAttnError(f"{name} failed ({rc}): {msg}")


def ptr(t) -> int | None:
    return None if t is None else t.data_ptr()


def stream(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def abi_version() -> int:
    return LIB.solattn_abi_version()
