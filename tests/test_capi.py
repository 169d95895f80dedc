"""The C ABI without a GPU: the library loads, exports every symbol that
include/solattn.h declares with the binding's signatures, rejects bad
arguments with error codes (no device work is reached), and its host-side
helpers (Morton, workspace sizing) answer correctly."""

import ctypes
import os
import re

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "solattn.h")


def declared():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(solattn_\w+)\s*\(", text)))


@pytest.fixture(scope="module")
def capi(pkg):
    import importlib
    return importlib.import_module(f"{pkg.__name__}._capi")


def test_exports_every_declared_symbol(capi):
    names = declared()
    assert len(names) >= 14
    for name in names:
        assert hasattr(capi.LIB, name), name
    assert set(names) == set(capi.SIGNATURES), "binding and header disagree"


def test_abi_version(capi):
    assert capi.abi_version() >> 16 == 2  # 2: routing masks only, no int16 block lists
    assert capi.abi_version() & 0xFFFF >= 1  # 2.1: int8_pv = SOLATTN_PV_INT8_RUNNING


def test_errors_are_reported(capi):
    L = capi.LIB
    null = None
    # head_dim 64 on the device path: rejected before any launch
    rc = L.solattn_pool(null, 0, 0, 0, null, 0, 0, 0, null, 0, 0, 0, 1, 100, 1, 64, 64,
                        null, null, 64, null, null, null)
    assert rc == -2 and b"head_dim" in L.solattn_last_error()
    rc = L.solattn_fwd_bf16(*([null, 0, 0, 0] * 3), null, null, 64, null, null,
                            1, 100, 1, 128, 96, 0.1, null, 0, 0, 0, null)
    assert rc == -2 and b"block" in L.solattn_last_error()
    rc = L.solattn_route(null, null, 1, null, null, 1, 10, 1, 128, 64, 0.1, 1.0, 0, 0, 0, 0, 0,
                         null, null, null, null)
    assert rc == -1
    # more than 16384 query blocks: rejected as unsupported (the node keeps such calls dense)
    rc = L.solattn_fwd_bf16(*([null, 0, 0, 0] * 3), null, null, 16448, null, null,
                            1, 16385 * 64, 1, 128, 64, 0.1, null, 0, 0, 0, null)
    assert rc == -2 and b"exceed" in L.solattn_last_error()
    rc = L.solattn_route(null, null, 16448, null, null, 1, 16385 * 64, 1, 128, 64, 0.1, 1.0, 0,
                         0, 0, 0, 0, null, null, null, null)
    assert rc == -2 and b"exceed" in L.solattn_last_error()
    # the pool's buffer offsets are 32-bit: token strides of 2^26 elements and more,
    # and more than 65535 spans of 128 tokens, are unsupported (no device work)
    fake = 1 << 20  # 16-byte aligned, never dereferenced
    big = 1 << 26
    rc = L.solattn_pool(fake, big * 8, big, 128, fake, 0, 128, 0, fake, 0, 128, 0, 1, 4, 1, 128,
                        128, fake, fake, 1, fake, null, null)
    assert rc == -2 and b"token strides" in L.solattn_last_error()
    rc = L.solattn_pool(fake, 0, 128, 0, fake, 0, 128, 0, fake, 0, 128, 0, 1, 65536 * 128, 1,
                        128, 128, fake, fake, 65536, fake, null, null)
    assert rc == -2 and b"tokens" in L.solattn_last_error()
    rc = L.solattn_moments(fake, 4, 1, 4, 32768, 128, 1, fake, fake, fake, fake, null)
    assert rc == -2 and b"heads" in L.solattn_last_error()
    with pytest.raises(capi.SolAttnError, match="null pointer"):
        capi.call("solattn_reorder_rows", null, 1, 0, 16, null, 0, 16, 1, 1, 16, null, null)
    ws = L.solattn_sol_attn_workspace_bytes(1, 1000, 2, 128, 64, 0)
    rc = L.solattn_sol_attn(*([null, 0, 0, 0] * 3), 1, 1000, 2, 128, 64, 0.1, 1.0, 0, 0, 0, 0,
                            null, ws - 1, null, 0, 0, 0, null)
    assert rc == -4 and b"workspace" in L.solattn_last_error()


def test_quant_block_variant_rejects_bad_arguments(capi, pkg):
    """The per-128-token-block INT8 variant: the C entry points refuse a short
    workspace and a head dim they do not take before any device work, and the
    Python options accept only quant_block None or 128."""
    import importlib
    import torch
    L = capi.LIB
    null = None
    ws = L.solattn_sol_attn_workspace_bytes(1, 1000, 2, 128, 128, 1)
    rc = L.solattn_sol_attn_int8_qblock(*([null, 0, 0, 0] * 3), 1, 1000, 2, 128, 128, 0.1, 1.0,
                                        0, 0, 0, 0, 1, null, ws - 1, null, 0, 0, 0, null)
    assert rc == -4 and b"workspace" in L.solattn_last_error()
    rc = L.solattn_quant_rows_blocked(null, 0, 0, 0, 1, 100, 1, 64, null, null, null, 100, null)
    assert rc == -2 and b"head_dim" in L.solattn_last_error()
    assert capi.QUANT_BLOCK == 128
    x = torch.zeros(1, 256, 2, 128, dtype=torch.bfloat16)
    i8 = importlib.import_module(f"{pkg.__name__}._int8_fwd")
    fp = importlib.import_module(f"{pkg.__name__}._fused_prep")
    for bad in (64, 256, 0):
        with pytest.raises(ValueError, match="quant_block"):
            i8.sol_attn_int8(x, x, x, tau=0.9, quant_block=bad)
        with pytest.raises(ValueError, match="quant_block"):
            fp.fused_preprocess_routing(x, x, x, tau=0.9, scale=0.1, quant_block=bad)


def test_int8_pv_modes(capi, pkg):
    """int8_pv takes the three SOLATTN_PV_* modes (bf16, block-max codes,
    running-max codes): another value is refused before any launch (stand-in
    addresses, never dereferenced), and the Python option maps onto them."""
    import importlib
    L = capi.LIB
    hdr = open(HEADER).read()
    for name, val in (("SOLATTN_PV_BF16", 0), ("SOLATTN_PV_INT8", 1), ("SOLATTN_PV_INT8_RUNNING", 2)):
        assert f"{name} = {val}" in hdr
    a = 1 << 20
    T, H = 1000, 2
    st, sb = H * 128, 1000 * H * 128
    for bad in (3, -1):
        args = [a, sb, st, 128, a, a, a, a, a, a, a, sb, st, 128, T, a, a, 64, a, a, 1, T, H, 128,
                64, 0.1, bad, a, sb, st, 128, None]
        rc = L.solattn_fwd_int8(*args)
        assert rc == -1 and b"SOLATTN_PV" in L.solattn_last_error()
        ws = L.solattn_sol_attn_workspace_bytes(1, T, H, 128, 64, 1)
        rc = L.solattn_sol_attn_int8(*([a, sb, st, 128] * 3), 1, T, H, 128, 64, 0.1, 1.0, 0, 0, 0,
                                     0, bad, a, ws, a, sb, st, 128, None)
        assert rc == -1 and b"SOLATTN_PV" in L.solattn_last_error()
    i8 = importlib.import_module(f"{pkg.__name__}._int8_fwd")
    assert i8._pv_mode(True, "block") == 1 and i8._pv_mode(True, "running") == 2
    assert i8._pv_mode(False, "running") == 0
    with pytest.raises(ValueError, match="pv_codes"):
        i8._pv_mode(True, "tile")


def test_noalloc_rejects_oversize_before_device_work(capi):
    """The allocation-free pipeline refuses shapes whose intermediates exceed
    its fixed scratch, with SOLATTN_ESIZE, before it touches a device."""
    L = capi.LIB
    B, T, H, D, block = 1, 131072, 40, 128, 64
    assert L.solattn_sol_attn_workspace_bytes(B, T, H, D, block, 0) > capi.NOALLOC_SCRATCH_BYTES
    rc = L.solattn_sol_attn_noalloc(*([None, 0, 0, 0] * 3), B, T, H, D, block, 0.1, 1.0, 0, 0, 0,
                                    0, None, 0, 0, 0, None)
    assert rc == -4 and b"scratch" in L.solattn_last_error()
    # cfg-4-sized calls fit
    assert L.solattn_sol_attn_workspace_bytes(1, 75600, 40, 128, 128, 0) <= capi.NOALLOC_SCRATCH_BYTES
    hdr = open(HEADER).read()
    assert f"({capi.NOALLOC_SCRATCH_BYTES >> 20}ll << 20)" in hdr


def test_workspace_bytes(capi):
    L = capi.LIB
    b0 = L.solattn_sol_attn_workspace_bytes(1, 32760, 24, 128, 128, 0)
    b1 = L.solattn_sol_attn_workspace_bytes(1, 32760, 24, 128, 128, 1)
    NT, npad, W = 256, 256, 8
    floor = 2 * npad * 24 * 128 * 2 + 24 * NT * 128 * 4 + 24 * NT * W * 4
    assert b0 >= floor and b1 > b0 + 3 * 32760 * 24 * 128
    assert b0 % 256 == 0
    assert L.solattn_sol_attn_workspace_bytes(0, 10, 1, 128, 64, 0) == 0


def test_workspace_has_no_block_lists(capi):
    """Routing is carried by the bitmask alone (NT^2 bits per head): at the
    kernels' 16384 blocks per head the BF16 workspace is far below what
    int16 lists (NT^2 x 2 bytes per head, 512 MiB) would need on their own."""
    L = capi.LIB
    for block in (64, 128):
        NT = 16384
        T = NT * block
        ws = L.solattn_sol_attn_workspace_bytes(1, T, 1, 128, block, 0)
        lists = NT * NT * 2
        mask = NT * (NT // 32) * 4
        assert mask <= ws < lists / 10, (block, ws)


def test_fwd_rejects_misaligned_output(capi):
    """Output rows are written as 16-byte stores: an o that is only 8-byte
    aligned, or whose strides are not multiples of 8 elements, is refused
    before any launch (the pointers are never dereferenced)."""
    L = capi.LIB
    a = 1 << 20  # a 256-byte-aligned stand-in address; nothing is launched
    T, H = 1000, 2
    st, sb = H * 128, 1000 * H * 128
    args = lambda o, so_t: ([a, sb, st, 128] * 3 + [a, a, 64, a, a, 1, T, H, 128, 64, 0.1]  # noqa: E731
                            + [o, sb, so_t, 128, None])
    for o, so_t in ((a + 8, st), (a, st + 4)):
        rc = L.solattn_fwd_bf16(*args(o, so_t))
        assert rc == -1 and b"16-byte aligned" in L.solattn_last_error()
    int8 = [a, sb, st, 128, a, a, a, a, None, None, a, sb, st, 128, T, a, a, 64, a, a, 1, T, H,
            128, 64, 0.1, 0, a + 8, sb, st, 128, None]
    rc = L.solattn_fwd_int8(*int8)
    assert rc == -1 and b"16-byte aligned" in L.solattn_last_error()


def test_host_morton(capi):
    n = 3 * 4 * 5
    perm = np.empty(n, np.int64)
    inv = np.empty(n, np.int64)
    rc = capi.LIB.solattn_morton_perm(3, 4, 5, 0, 0, perm.ctypes.data, inv.ctypes.data)
    assert rc == 0
    assert np.array_equal(np.sort(perm), np.arange(n)) and np.array_equal(perm[inv], np.arange(n))
    assert capi.LIB.solattn_morton_perm(0, 4, 5, 0, 0, perm.ctypes.data, inv.ctypes.data) == -1
    assert capi.LIB.solattn_morton_perm(3, 4, 5, 7, 0, perm.ctypes.data, inv.ctypes.data) == -1


def test_product_does_not_import_oracle():
    """The package never imports or loads the oracle."""
    pkg_dir = os.path.join(ROOT, "comfyui-solattn_triton_amd")
    banned = re.compile(r"^\s*(import\s+oracle|from\s+oracle)|liboracle|oracle\.\w+\(", re.M)
    for dirpath, _, files in os.walk(pkg_dir):
        for f in files:
            if f.endswith((".py", ".hip", ".hpp", ".cpp")):
                src = open(os.path.join(dirpath, f)).read()
                assert not banned.search(src), f
