"""The bench's work accounting on the CPU: the routed-FLOP count behind
`roofline.achieved`, the exact/pooled split and the INT8 mixed-peak roofline,
against brute-force counts over small random routing masks."""

import math
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
import bench  # noqa: E402


def random_mask(B, H, NT, density, seed):
    """uint32 bitmask [B, H, NT, ceil(NT/32)] with the diagonal always set."""
    rng = np.random.default_rng(seed)
    ex = rng.random((B, H, NT, NT)) < density
    ex |= np.eye(NT, dtype=bool)[None, None]
    W = (NT + 31) // 32
    words = np.zeros((B, H, NT, W), dtype=np.uint64)
    for j in range(NT):
        words[..., j // 32] |= ex[..., j].astype(np.uint64) << np.uint64(j % 32)
    return ex, torch.from_numpy(words.astype(np.uint32).view(np.int32))


@pytest.mark.parametrize("T,block", [(1000, 64), (777, 128), (4096, 64), (2500, 128)])
def test_routed_flops_brute_force(T, block):
    B, H, D = 2, 3, 128
    NT = math.ceil(T / block)
    ex, mask = random_mask(B, H, NT, 0.3, T)
    lens = [min(block, T - block * j) for j in range(NT)]
    want_exact = want_pooled = 0
    for b in range(B):
        for h in range(H):
            for i in range(NT):
                for j in range(NT):
                    if ex[b, h, i, j]:
                        want_exact += 4 * D * lens[i] * lens[j]
                    else:
                        want_pooled += 4 * D * lens[i]
    counts = torch.from_numpy(ex.sum(-1).astype(np.int32))
    assert bench.routed_flops(counts, mask, T, block, D) == pytest.approx(want_exact + want_pooled, rel=1e-12)
    exact, pooled = bench.split_ops(counts, mask, T, block, D)
    assert exact == pytest.approx(want_exact, rel=1e-12)
    assert pooled == pytest.approx(want_pooled, rel=1e-12)


def test_dense_flops():
    assert bench.dense_flops(1, 24, 32760, 128) == pytest.approx(13.19e12, rel=1e-3)


def test_int8_roofline_mix():
    exact, pooled = 2.0e12, 0.1e12
    r = bench.int8_roofline(1.0, exact, pooled, int8_pv=False)
    ideal = 1e3 * (exact / 2 / 5000e12 + exact / 2 / 2500e12 + pooled / 2500e12)
    assert r["ideal_ms_at_peak"] == pytest.approx(ideal, rel=1e-3)
    assert r["frac"] == pytest.approx(ideal / 1.0, rel=1e-3)
    r8 = bench.int8_roofline(1.0, exact, pooled, int8_pv=True)
    assert r8["ideal_ms_at_peak"] < r["ideal_ms_at_peak"]
