"""Host-side check of the forward kernels' workgroup -> query-block mapping.

The forwards (``csrc/fwd_common.hpp``, ``tile_coords_lpt``) deal workgroups
to XCDs round-robin, give each XCD a contiguous run of query blocks, and
inside each window of 8192 query tokens (64 dispatches at block 128, 128 at
block 64) take the query blocks longest first. The
mapping must be a permutation of ``[0, grid)`` for every grid size and every
count pattern, or a query block is computed twice and another never (or an
index leaves the buffers). This restates the index arithmetic step by step
(fill the window, rank it, pick rank r) for the workgroup sizes the kernels
launch with and checks the permutation property, which the kernel's parity
tests only see for the grid sizes they run.
"""
import numpy as np
import pytest


def _mapping(counts, threads, WINDOW):
    total = len(counts)
    out = np.empty(total, dtype=np.int64)
    for w in range(total):
        if total % 8 == 0:
            per, li = total // 8, w // 8
            base = (w % 8) * per + (li & ~(WINDOW - 1))
            r = li & (WINDOW - 1)
            nwin = min(WINDOW, per - (li & ~(WINDOW - 1)))
        else:
            base = w & ~(WINDOW - 1)
            r = w & (WINDOW - 1)
            nwin = min(WINDOW, total - base)
        s_cnt = [-1] * WINDOW
        for t0 in range(threads):  # strided fill, as the kernel does
            for t in range(t0, WINDOW, threads):
                s_cnt[t] = counts[base + t] if t < nwin else -1
        pick = None
        for t0 in range(threads):
            for t in range(t0, nwin, threads):
                rank = sum((s_cnt[u] > s_cnt[t]) or (s_cnt[u] == s_cnt[t] and u < t)
                           for u in range(nwin))
                if rank == r:
                    assert pick is None, "two slots share a rank"
                    pick = t
        assert pick is not None, f"no slot has rank {r} (w={w})"
        out[w] = base + pick
    return out


@pytest.mark.parametrize("total", [1, 7, 8, 24, 63, 64, 65, 200, 512, 520, 1031, 2048 + 8])
@pytest.mark.parametrize("threads,window", [(256, 64), (128, 128), (128, 64), (256, 128)])
def test_dispatch_map_is_permutation(total, threads, window):
    rng = np.random.default_rng(total * 7 + threads)
    counts = rng.integers(0, 5, size=total).tolist()  # many ties
    m = _mapping(counts, threads, window)
    assert sorted(m.tolist()) == list(range(total))


@pytest.mark.parametrize("threads,WINDOW", [(256, 64), (128, 128)])
def test_dispatch_map_longest_first_within_window(threads, WINDOW):
    total = 8 * 256
    counts = list(range(total))  # strictly increasing: every window reverses
    m = _mapping(counts, threads, WINDOW)
    per = total // 8
    for xcd in range(8):
        for win in range(0, per, WINDOW):
            ws = [m[(li * 8) + xcd] for li in range(win, win + WINDOW)]
            got = [counts[i] for i in ws]
            assert got == sorted(got, reverse=True)
            assert sorted(ws) == list(range(xcd * per + win, xcd * per + win + WINDOW))
