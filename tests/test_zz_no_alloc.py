"""The allocation-free BF16 pipeline (solattn_sol_attn_noalloc) against the
workspace one (solattn_sol_attn): the same kernels over a fixed per-device
scratch array, so the outputs must be identical bit for bit. Two calls in a
row, the second on a smaller input, so a stale first call's intermediates in
the shared scratch would show; and the call captured in a HIP graph and
replayed on new inputs."""

import numpy as np
import pytest
import torch

from _util import bits, randn_bf16

pytestmark = pytest.mark.gpu


def _noalloc(capi, q, k, v, block, tau, sink_kv=(0, 0), sink_q=(0, 0)):
    B, T, H, D = q.shape
    out = torch.empty((B, T, H, D), device=q.device, dtype=torch.bfloat16)
    with torch.cuda.device(q.device):
        capi.call("solattn_sol_attn_noalloc", q.data_ptr(), *q.stride()[:3], k.data_ptr(),
                  *k.stride()[:3], v.data_ptr(), *v.stride()[:3], B, T, H, D, block,
                  float(D ** -0.5), float(tau), int(sink_kv[0]), int(sink_kv[1]), int(sink_q[0]),
                  int(sink_q[1]), out.data_ptr(), *out.stride()[:3], capi.stream(q.device))
    return out


@pytest.mark.parametrize("block", [64, 128])
def test_noalloc_matches_workspace_entry(pkg, dev, block):
    import importlib
    capi = importlib.import_module(f"{pkg.__name__}._capi")
    tri = importlib.import_module(f"{pkg.__name__}._tri_fwd")
    # a large call, then a smaller one with a different head count and sinks
    cases = [((1, 4100, 6, 128), 0.9, (0, 0), (0, 0), 20),
             ((2, 777, 3, 128), 0.5, (0, 2), (0, 1), 30)]
    for shape, tau, skv, sq, seed in cases:
        print(f"[noalloc] block={block} shape={shape} tau={tau} sink_kv={skv} sink_q={sq}",
              flush=True)
        q, k, v = (randn_bf16(shape, seed + i).to(dev) for i in range(3))
        ref = tri.sol_attn(q, k, v, tau=tau, block=block, sink_blocks=skv, sink_q=sq)
        got = _noalloc(capi, q, k, v, block, tau, skv, sq)
        torch.cuda.synchronize()
        assert np.array_equal(bits(got), bits(ref)), f"noalloc differs at {shape}"


def test_noalloc_replays_under_hip_graph(pkg, dev):
    """The use the entry exists for: captured once into a HIP graph (torch's
    capture stream; nothing is allocated or memset inside the capture), then
    replayed on new inputs copied into the captured buffers, with eager work
    and a synchronisation between replays. Every replay equals the workspace
    entry point's eager result bit for bit."""
    import importlib
    capi = importlib.import_module(f"{pkg.__name__}._capi")
    tri = importlib.import_module(f"{pkg.__name__}._tri_fwd")
    shape, block, tau = (1, 2000, 4, 128), 128, 0.9
    q, k, v = (randn_bf16(shape, 60 + i).to(dev) for i in range(3))
    out = torch.empty(shape, device=dev, dtype=torch.bfloat16)
    B, T, H, D = shape

    def launch():
        capi.call("solattn_sol_attn_noalloc", q.data_ptr(), *q.stride()[:3], k.data_ptr(),
                  *k.stride()[:3], v.data_ptr(), *v.stride()[:3], B, T, H, D, block,
                  float(D ** -0.5), float(tau), 0, 0, 0, 0, out.data_ptr(), *out.stride()[:3],
                  capi.stream(dev))

    launch()  # first use on this device resolves the scratch array, outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        launch()
    for rep in range(3):
        print(f"[noalloc graph] replay {rep}", flush=True)
        for i, t in enumerate((q, k, v)):
            t.copy_(randn_bf16(shape, 70 + 10 * rep + i).to(dev))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        ref = tri.sol_attn(q, k, v, tau=tau, block=block)
        torch.cuda.synchronize()
        assert np.array_equal(bits(out), bits(ref)), f"replay {rep} differs"


def test_noalloc_rejects_oversize(pkg, dev):
    import importlib
    capi = importlib.import_module(f"{pkg.__name__}._capi")
    B, T, H, D, block = 1, 131072, 40, 128, 64  # intermediates far beyond the scratch
    need = capi.LIB.solattn_sol_attn_workspace_bytes(B, T, H, D, block, 0)
    assert need > capi.NOALLOC_SCRATCH_BYTES
    q = torch.empty((1, 8, 1, 128), device=dev, dtype=torch.bfloat16)
    with pytest.raises(capi.SolAttnError, match="scratch"):
        capi.call("solattn_sol_attn_noalloc", q.data_ptr(), 0, 0, 0, q.data_ptr(), 0, 0, 0,
                  q.data_ptr(), 0, 0, 0, B, T, H, D, block, 0.1, 1.0, 0, 0, 0, 0, q.data_ptr(),
                  0, 0, 0, capi.stream(dev))
