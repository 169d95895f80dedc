"""GPU parity at the benchmark's full size (config 2: B=1, H=24, D=128,
N=32760 from a 21x30x52 latent grid, Morton-reordered, tau 0.9; the same
synthetic smooth-field inputs ``bench.py`` times), at block 128 (the
benchmark's) and block 64.

The permutation and the whole routing state (pooled keys, thresholds, counts,
bitmask and the exact lists it encodes) are compared with the oracle bit for bit over every head and
query block; the forward outputs are compared with the oracle's restatement of
the reference loop on a seeded sample of query blocks (the oracle is a scalar
loop; 96 BF16 and 32 INT8 query blocks take seconds). The small-case tests
cover ragged tails, sinks and edge sizes; these cover the sizes the kernels are measured at
(grids of 6144 and 12288 workgroups, 256 and 512 blocks per head, the
dispatch windows).
"""

import importlib

import numpy as np
import pytest
import torch

import bench
import oracle
from _util import bits, check_int8_blocks, compare_rows, mask_bits, u32

pytestmark = pytest.mark.gpu

BF16_MAXABS, BF16_COS = 2e-2, 0.9995


def _inputs(pkg, dev, config):
    """Inputs of a bench config, Morton-reordered on the GPU, plus their bf16
    bits on the host."""
    mort = importlib.import_module(f"{pkg.__name__}._morton")
    cfg = dict(bench.CONFIGS[config])
    print(f"[full size] cfg{config} grid={cfg['grid']} H={cfg['H']}", flush=True)
    q, k, v = bench.make_inputs(cfg, dev)
    perm, inv = mort.morton_perm(cfg["grid"], dev, "3d")
    ref_perm, ref_inv = oracle.morton_perm(cfg["grid"], "3d")
    assert np.array_equal(perm.cpu().numpy(), ref_perm)
    assert np.array_equal(inv.cpu().numpy(), ref_inv)
    q, k, v = (mort.reorder_tokens(t, perm, dim=1) for t in (q, k, v))
    torch.cuda.synchronize()
    return cfg, (q, k, v), tuple(bits(t) for t in (q, k, v))


@pytest.fixture(scope="module")
def video(pkg, dev):
    return _inputs(pkg, dev, 2)


def _route_equal(r, ref):
    B, H, NT = ref["counts"].shape
    assert np.array_equal(bits(r.kc), ref["kc"])
    assert np.array_equal(bits(r.vc), ref["vc"])
    assert np.array_equal(r.threshold.cpu().numpy().view(np.uint32), ref["thr"].view(np.uint32))
    assert np.array_equal(r.counts.cpu().numpy(), ref["counts"])
    assert np.array_equal(u32(r.mask), ref["mask"])
    # the ascending exact lists the forwards build from the mask rows
    ex = mask_bits(u32(r.mask), NT)
    assert np.array_equal(ex.sum(-1), ref["counts"])
    n = ref["counts"]
    valid = np.arange(NT)[None, None, None, :] < n[..., None]
    order = np.argsort(~ex, axis=-1, kind="stable")  # exact blocks first, ascending
    assert np.array_equal(np.where(valid, order, 0), np.where(valid, ref["lists"], 0))


def _near_ties(ref, ulps=8):
    """Routing decisions within ``ulps`` ulps of the threshold: the ones another
    summation order of the same scores (the reference's MMA) could flip.
    Reported, not asserted; the build's own decisions are bit-exact above."""
    s, t = ref["scores"], np.transpose(ref["thr"], (0, 2, 1))[..., None]
    mag = np.maximum(np.abs(s), np.abs(t)).astype(np.float32)
    return int((np.abs(s - t) <= ulps * np.spacing(mag)).sum()), s.size


def _sample_rows(H, NT, n, seed):
    rng = np.random.default_rng(seed)
    picks = sorted(rng.choice(H * NT, n, replace=False))
    return [(0, int(p) // NT, int(p) % NT) for p in picks]


@pytest.mark.parametrize("block", [128, 64])
def test_full_size_bf16(pkg, dev, video, block):
    pre = importlib.import_module(f"{pkg.__name__}._preprocess")
    tri = importlib.import_module(f"{pkg.__name__}._tri_fwd")
    cfg, (q, k, v), (qb, kb, vb) = video
    tau = cfg["tau"]
    r = pre.route(q, k, v, scale=128 ** -0.5, tau=tau, block=block)
    out = tri.sol_attn(q, k, v, tau=tau, block=block)
    torch.cuda.synchronize()
    ref = oracle.prepare(qb, kb, vb, block=block, tau=tau, want_scores=True)
    _route_equal(r, ref)
    density = float(ref["counts"].sum()) / ref["counts"].size / ref["NT"]
    ties, pairs = _near_ties(ref)
    print(f"[full size bf16 block {block}] routing bit-exact, exact-block density "
          f"{density:.3f}; {ties} of {pairs} decisions within 8 ulp of the threshold", flush=True)
    rows = _sample_rows(cfg["H"], ref["NT"], 96, seed=5)
    port = oracle.forward_port(qb, kb, vb, ref, rows)
    got = out.float().cpu().numpy()
    err, cos = compare_rows(got, port, block)
    worst = min(cosine_rows(got, port, block))
    print(f"[full size bf16 block {block}] {len(rows)} query blocks: max|err|={err:.3e} "
          f"cos={cos:.6f}, worst block cos {worst:.6f}", flush=True)
    assert err < BF16_MAXABS and cos >= BF16_COS and worst >= BF16_COS


INT8_CASES = [  # (block, tau): BASELINE config 3 sweeps tau at block 128
    (128, 0.8), (128, 0.9), (128, 0.95), (64, 0.9)]


@pytest.mark.parametrize("block,tau", INT8_CASES)
@pytest.mark.parametrize("int8_pv", [True, False])
def test_full_size_int8(pkg, dev, video, int8_pv, block, tau):
    fp = importlib.import_module(f"{pkg.__name__}._fused_prep")
    i8 = importlib.import_module(f"{pkg.__name__}._int8_fwd")
    cfg, (q, k, v), (qb, kb, vb) = video
    r, qi, qs, ki, ks, vi = fp.fused_preprocess_routing(q, k, v, tau=tau, scale=128 ** -0.5,
                                                        block=block)
    out = i8.forward_int8(q, v, r, qi, qs, ki, ks, vi, int8_pv=int8_pv)
    # the one-call pipeline (Q codes from the pooling pass, K and V codes from
    # the quantisation pass) feeds the same forward the same bits
    one = i8.sol_attn_int8(q, k, v, tau=tau, block=block, int8_pv=int8_pv)
    torch.cuda.synchronize()
    assert torch.equal(one.view(torch.int16), out.view(torch.int16))
    ref = oracle.prepare(qb, kb, vb, block=block, tau=tau, int8=True, int8_pv=int8_pv)
    _route_equal(r, ref)
    T = ref["T"]
    assert np.array_equal(qi[:, :T].cpu().numpy(), ref["qi"][:, :T])
    assert np.array_equal(ki[:, :T].cpu().numpy(), ref["ki"][:, :T])
    assert np.array_equal(qs[:, :T].cpu().numpy().view(np.uint32), ref["qs"][:, :T].view(np.uint32))
    assert np.array_equal(ks[:, :T].cpu().numpy().view(np.uint32), ref["ks"][:, :T].view(np.uint32))
    if int8_pv:
        assert np.array_equal(vi[:, :T].cpu().numpy(), ref["vi"][:, :T])
        assert np.array_equal(r.vscale.cpu().numpy().view(np.uint32), ref["vscale"].view(np.uint32))
    density = float(ref["counts"].sum()) / ref["counts"].size / ref["NT"]
    print(f"[full size int8 block {block} tau {tau} pv={int8_pv}] routing and codes bit-exact, "
          f"exact-block density {density:.3f}", flush=True)
    NT = ref["NT"]
    rows = sorted(set(_sample_rows(cfg["H"], NT, 32, seed=6)) | {(0, 0, NT - 1), (0, 23, NT - 1)})
    check_int8_blocks(f"full size int8 block {block} tau {tau} pv={int8_pv}",
                      out.float().cpu().numpy(), qb, vb, ref, rows, int8_pv, block)
    if int8_pv:  # the running-max codes on the same routing and codes
        run = i8.forward_int8(q, v, r, qi, qs, ki, ks, vi, pv_codes="running")
        one = i8.sol_attn_int8(q, k, v, tau=tau, block=block, pv_codes="running")
        torch.cuda.synchronize()
        assert torch.equal(one.view(torch.int16), run.view(torch.int16))
        check_int8_blocks(f"full size int8 block {block} tau {tau} running codes",
                          run.float().cpu().numpy(), qb, vb, ref, rows, True, block,
                          pv_codes="running")


@pytest.mark.parametrize("int8_pv", [True, False])
def test_full_size_int8_quant_block(pkg, dev, video, int8_pv):
    """BASELINE config 3's wording, Q/K quantised per 128-token block, at full
    size: codes and scales bit-exact, routing unchanged, forward per query block
    against the oracle loops fed the same codes."""
    fp = importlib.import_module(f"{pkg.__name__}._fused_prep")
    i8 = importlib.import_module(f"{pkg.__name__}._int8_fwd")
    cfg, (q, k, v), (qb, kb, vb) = video
    block, tau = 128, cfg["tau"]
    r, qi, qs, ki, ks, vi = fp.fused_preprocess_routing(q, k, v, tau=tau, scale=128 ** -0.5,
                                                        block=block, quant_block=128)
    out = i8.sol_attn_int8(q, k, v, tau=tau, block=block, int8_pv=int8_pv, quant_block=128)
    torch.cuda.synchronize()
    ref = oracle.prepare(qb, kb, vb, block=block, tau=tau, int8=True, int8_pv=int8_pv,
                         quant_block=128)
    _route_equal(r, ref)
    T = ref["T"]
    assert np.array_equal(qi[:, :T].cpu().numpy(), ref["qi"][:, :T])
    assert np.array_equal(ki[:, :T].cpu().numpy(), ref["ki"][:, :T])
    assert np.array_equal(qs[:, :T].cpu().numpy().view(np.uint32), ref["qs"][:, :T].view(np.uint32))
    assert np.array_equal(ks[:, :T].cpu().numpy().view(np.uint32), ref["ks"][:, :T].view(np.uint32))
    print(f"[full size int8 quant_block 128 pv={int8_pv}] routing and codes bit-exact", flush=True)
    NT = ref["NT"]
    rows = sorted(set(_sample_rows(cfg["H"], NT, 32, seed=7)) | {(0, 0, NT - 1)})
    check_int8_blocks(f"full size int8 quant_block pv={int8_pv}", out.float().cpu().numpy(), qb,
                      vb, ref, rows, int8_pv, block)


@pytest.fixture(scope="module")
def image(pkg, dev):
    cfg = dict(bench.CONFIGS[1])
    print(f"[full size] cfg1 grid={cfg['grid']} H={cfg['H']} (no reordering)", flush=True)
    q, k, v = bench.make_inputs(cfg, dev)
    torch.cuda.synchronize()
    return cfg, (q, k, v), tuple(bits(t) for t in (q, k, v))


def test_cfg1_image_dit_bf16(pkg, dev, image):
    """BASELINE config 1 (H24, N 4096 from a 1x64x64 grid, block 64, per-head K
    offset, tau 0.9): routing bit-exact and every one of the 1536 query blocks
    against the reference loop."""
    pre = importlib.import_module(f"{pkg.__name__}._preprocess")
    tri = importlib.import_module(f"{pkg.__name__}._tri_fwd")
    cfg, (q, k, v), (qb, kb, vb) = image
    block, tau = cfg["block"], cfg["tau"]
    r = pre.route(q, k, v, scale=128 ** -0.5, tau=tau, block=block)
    out = tri.sol_attn(q, k, v, tau=tau, block=block)
    torch.cuda.synchronize()
    ref = oracle.prepare(qb, kb, vb, block=block, tau=tau, want_scores=True)
    _route_equal(r, ref)
    ties, pairs = _near_ties(ref)
    rows = [(0, h, i) for h in range(cfg["H"]) for i in range(ref["NT"])]
    port = oracle.forward_port(qb, kb, vb, ref, rows)
    err, cos = compare_rows(out.float().cpu().numpy(), port, block)
    worst = min(cosine_rows(out.float().cpu().numpy(), port, block))
    print(f"[cfg1 bf16] routing bit-exact ({ties} of {pairs} decisions within 8 ulp); "
          f"{len(rows)} query blocks: max|err|={err:.3e} cos={cos:.6f}, worst block cos "
          f"{worst:.6f}", flush=True)
    assert err < BF16_MAXABS and cos >= BF16_COS and worst >= BF16_COS


@pytest.mark.parametrize("int8_pv", [True, False])
def test_cfg1_image_dit_int8(pkg, dev, image, int8_pv):
    fp = importlib.import_module(f"{pkg.__name__}._fused_prep")
    i8 = importlib.import_module(f"{pkg.__name__}._int8_fwd")
    cfg, (q, k, v), (qb, kb, vb) = image
    block, tau = cfg["block"], cfg["tau"]
    r, qi, qs, ki, ks, vi = fp.fused_preprocess_routing(q, k, v, tau=tau, scale=128 ** -0.5,
                                                        block=block)
    out = i8.forward_int8(q, v, r, qi, qs, ki, ks, vi, int8_pv=int8_pv)
    # the one-call pipeline (Q codes from the pooling pass, K and V codes from
    # the quantisation pass) feeds the same forward the same bits
    one = i8.sol_attn_int8(q, k, v, tau=tau, block=block, int8_pv=int8_pv)
    torch.cuda.synchronize()
    assert torch.equal(one.view(torch.int16), out.view(torch.int16))
    ref = oracle.prepare(qb, kb, vb, block=block, tau=tau, int8=True, int8_pv=int8_pv)
    _route_equal(r, ref)
    assert np.array_equal(qi.cpu().numpy(), ref["qi"]) and np.array_equal(ki.cpu().numpy(), ref["ki"])
    if int8_pv:
        assert np.array_equal(vi.cpu().numpy(), ref["vi"])
    rows = [(0, h, i) for h in range(cfg["H"]) for i in range(ref["NT"])]
    if not int8_pv:
        rows = rows[::3]  # the bf16-P.V loop is the slower one on the host
    check_int8_blocks(f"cfg1 int8 pv={int8_pv}", out.float().cpu().numpy(), qb, vb, ref, rows,
                      int8_pv, block)
    if int8_pv:  # the running-max codes on the same routing and codes
        run = i8.forward_int8(q, v, r, qi, qs, ki, ks, vi, pv_codes="running")
        check_int8_blocks("cfg1 int8 running codes", run.float().cpu().numpy(), qb, vb, ref, rows,
                          True, block, pv_codes="running")


def cosine_rows(got, port, block):
    from _util import per_block
    return [s[2] for s in per_block(got, port, block)]


def test_full_size_long_video(pkg, dev):
    """cfg 4 (B=1, H=40, N=75600 from 21x60x60, block 128: 591 blocks per head,
    an 80-token last block, a grid of 23640 workgroups), the whole pipeline:
    Morton reorder -> routing (bit-exact over every query block) -> BF16 and
    INT8 forwards (int8 P.V, bf16 P.V and the per-128-token-block variant) on
    sampled query blocks, including the ragged last one, against the oracle
    loops -> inverse reorder of the output, against the oracle's inverse."""
    pre = importlib.import_module(f"{pkg.__name__}._preprocess")
    tri = importlib.import_module(f"{pkg.__name__}._tri_fwd")
    fp = importlib.import_module(f"{pkg.__name__}._fused_prep")
    i8 = importlib.import_module(f"{pkg.__name__}._int8_fwd")
    mort = importlib.import_module(f"{pkg.__name__}._morton")
    cfg, (q, k, v), (qb, kb, vb) = _inputs(pkg, dev, 4)
    block, tau = cfg["block"], cfg["tau"]
    r = pre.route(q, k, v, scale=128 ** -0.5, tau=tau, block=block)
    out = tri.sol_attn(q, k, v, tau=tau, block=block)
    # inverse reorder of the output back to raster order (the pipeline's last step)
    _, inv = mort.morton_perm(cfg["grid"], dev, "3d")
    back = mort.reorder_tokens(out, inv, dim=1)
    torch.cuda.synchronize()
    _, ref_inv = oracle.morton_perm(cfg["grid"], "3d")
    assert np.array_equal(bits(back), bits(out)[:, ref_inv])
    del back
    ref = oracle.prepare(qb, kb, vb, block=block, tau=tau)
    _route_equal(r, ref)
    NT = ref["NT"]
    rows = _sample_rows(cfg["H"], NT, 32, seed=7) + [(0, 0, NT - 1), (0, cfg["H"] - 1, NT - 1)]
    port = oracle.forward_port(qb, kb, vb, ref, rows)
    got = out.float().cpu().numpy()
    err, cos = compare_rows(got, port, block)
    worst = min(cosine_rows(got, port, block))
    print(f"[full size cfg4 bf16] routing bit-exact, inverse reorder bit-exact; {len(rows)} "
          f"query blocks: max|err|={err:.3e} cos={cos:.6f}, worst block cos {worst:.6f}",
          flush=True)
    assert err < BF16_MAXABS and cos >= BF16_COS and worst >= BF16_COS
    del out, port, ref, got
    r8, qi, qs, ki, ks, vi = fp.fused_preprocess_routing(q, k, v, tau=tau, scale=128 ** -0.5,
                                                         block=block)
    ref8 = oracle.prepare(qb, kb, vb, block=block, tau=tau, int8=True, int8_pv=True)
    _route_equal(r8, ref8)
    T = ref8["T"]
    for name, mine in (("qi", qi), ("ki", ki), ("vi", vi)):
        assert np.array_equal(mine[:, :T].cpu().numpy(), ref8[name][:, :T]), name
    rows8 = rows[::3] + rows[-2:]
    for pv, codes in ((True, "block"), (True, "running"), (False, "block")):
        out8 = i8.forward_int8(q, v, r8, qi, qs, ki, ks, vi, int8_pv=pv, pv_codes=codes)
        one = i8.sol_attn_int8(q, k, v, tau=tau, block=block, int8_pv=pv, pv_codes=codes)
        torch.cuda.synchronize()
        assert torch.equal(one.view(torch.int16), out8.view(torch.int16))
        check_int8_blocks(f"full size cfg4 int8 pv={pv} {codes}", out8.float().cpu().numpy(), qb,
                          vb, ref8, rows8, pv, block, pv_codes=codes)
        del out8, one
    del r8, qi, qs, ki, ks, vi, ref8
    outb = i8.sol_attn_int8(q, k, v, tau=tau, block=block, int8_pv=True, quant_block=128)
    refb = oracle.prepare(qb, kb, vb, block=block, tau=tau, int8=True, int8_pv=True,
                          quant_block=128)
    torch.cuda.synchronize()
    check_int8_blocks("full size cfg4 int8 quant_block 128", outb.float().cpu().numpy(), qb, vb,
                      refb, rows8, True, block)
