"""Golden fixtures (tests/golden/*.npz, written by make_golden.py): the CPU
oracle must still reproduce them bit for bit; the HIP kernels must match them
(bit-exact prep/routing/quant, forward within the BF16 / INT8 tolerances)."""

import glob
import os

import numpy as np
import pytest
import torch

import oracle
from _util import check_int8_blocks, cosine, from_bits, u32

FIXTURES = sorted(glob.glob(os.path.join(os.path.dirname(__file__), "golden", "*.npz")))


def _load(path):
    return dict(np.load(path, allow_pickle=False))


@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_oracle_reproduces_golden(path):
    g = _load(path)
    int8 = bool(g["int8"])
    p = oracle.prepare(g["q"], g["k"], g["v"], block=int(g["block"]), tau=float(g["tau"]),
                       int8=int8, sink_kv=tuple(g["sink_kv"]), sink_q=tuple(g["sink_q"]))
    NT = p["NT"]
    for key in ("kc", "vc"):
        assert np.array_equal(p[key][:, :NT], g[key]), key
    for key in ("counts", "mask"):
        assert np.array_equal(p[key], g[key]), key
    for key in ("qbar", "kc_mean", "kc_var", "thr"):
        assert np.array_equal(p[key].view(np.uint32), g[key].view(np.uint32)), key
    if int8:
        for key in ("qi", "ki", "vi"):
            assert np.array_equal(p[key], g[key]), key
        for key in ("qs", "ks", "vscale"):
            assert np.array_equal(p[key].view(np.uint32), g[key].view(np.uint32)), key
    rows = [(0, h, i) for h in range(int(g["H"])) for i in range(p["NT"])]
    fwd = (oracle.forward_int8_port(g["q"], g["v"], p, rows) if int8
           else oracle.forward_port(g["q"], g["k"], g["v"], p, rows))
    out = np.concatenate([fwd[r] for r in rows]).reshape(int(g["H"]), -1, 128)[:, :int(g["T"])]
    assert np.array_equal(out.astype(np.float16), g["out"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", FIXTURES, ids=os.path.basename)
def test_gpu_matches_golden(pkg, dev, path):
    import importlib
    g = _load(path)
    n = pkg.__name__
    prep = importlib.import_module(f"{n}._preprocess")
    tri = importlib.import_module(f"{n}._tri_fwd")
    i8 = importlib.import_module(f"{n}._int8_fwd")
    q, k, v = (from_bits(g[x], dev) for x in ("q", "k", "v"))
    int8, block, tau = bool(g["int8"]), int(g["block"]), float(g["tau"])
    skv, sq = tuple(int(x) for x in g["sink_kv"]), tuple(int(x) for x in g["sink_q"])
    print(f"[golden] {os.path.basename(path)}", flush=True)
    r = prep.route(q, k, v, scale=128 ** -0.5, tau=tau, block=block, int8=int8, v_absmax=int8,
                   sink_blocks=skv, sink_q=sq)
    NT = g["counts"].shape[-1]
    assert np.array_equal(r.kc[:, :NT].cpu().view(torch.int16).numpy().view(np.uint16), g["kc"])
    assert np.array_equal(r.threshold.cpu().numpy().view(np.uint32), g["thr"].view(np.uint32))
    assert np.array_equal(u32(r.mask), g["mask"])
    assert np.array_equal(r.counts.cpu().numpy(), g["counts"])
    if int8:
        out = i8.sol_attn_int8(q, k, v, tau=tau, block=block, sink_blocks=skv, sink_q=sq)
    else:
        out = tri.sol_attn(q, k, v, tau=tau, block=block, sink_blocks=skv, sink_q=sq)
    got = out.float().cpu().numpy()[0].transpose(1, 0, 2)  # [H, T, D]
    ref = g["out"].astype(np.float32)
    if int8:
        assert cosine(got, ref) >= 0.999
        # per query block, against the reference and the kernel arithmetic
        p = oracle.prepare(g["q"], g["k"], g["v"], block=block, tau=tau, int8=True,
                           sink_kv=skv, sink_q=sq)
        rows = [(0, h, i) for h in range(int(g["H"])) for i in range(NT)]
        check_int8_blocks(f"golden {os.path.basename(path)}", out.float().cpu().numpy(), g["q"],
                          g["v"], p, rows, True, block)
    else:
        assert np.abs(got - ref).max() < 2e-2 and cosine(got, ref) >= 0.9995
