"""Pins of the CPU oracle (no GPU): every oracle function is checked against
something the mathematics fixes -- brute force, closed forms in float64,
textbook orders, hand-built cases -- chosen so that a dropped term, a wrong
index or a transposed operand fails."""

import math

import numpy as np
import pytest
import torch

import oracle
from _util import bits, cosine, randn_bf16


# ------------------------------------------------------------------ Morton
def _interleave(x, y, z):
    """Bit loop: bit i of x -> 3i, of y -> 3i+1, of z -> 3i+2."""
    code = 0
    for i in range(21):
        code |= ((x >> i) & 1) << (3 * i) | ((y >> i) & 1) << (3 * i + 1) | ((z >> i) & 1) << (3 * i + 2)
    return code


def _brute_perm(grid, curve):
    f, h, w = grid
    keys = []
    for lin in range(f * h * w):
        z, rem = divmod(lin, h * w)
        y, x = divmod(rem, w)
        if curve == "2d_frame":
            key = (z << 42) | _interleave(x, y, 0)
        else:
            key = _interleave(x, y, z)
        keys.append((key, lin))
    return np.array([lin for _, lin in sorted(keys)], np.int64)


@pytest.mark.parametrize("grid", [(2, 2, 2), (3, 5, 7), (4, 4, 4), (1, 6, 10), (5, 3, 9)])
@pytest.mark.parametrize("curve", ["3d", "2d_frame"])
def test_morton_brute_force(grid, curve):
    perm, inv = oracle.morton_perm(grid, curve)
    assert np.array_equal(perm, _brute_perm(grid, curve))
    assert np.array_equal(perm[inv], np.arange(perm.size))
    assert np.array_equal(inv[perm], np.arange(perm.size))


def test_morton_known_answers():
    # 2x2x2: Z-order of a unit cube is the raster order (x fastest, then y, then t).
    assert np.array_equal(oracle.morton_perm((2, 2, 2))[0], np.arange(8))
    # 4x4 single frame: the textbook 2-D Z curve.
    z4 = [0, 1, 4, 5, 2, 3, 6, 7, 8, 9, 12, 13, 10, 11, 14, 15]
    assert np.array_equal(oracle.morton_perm((1, 4, 4))[0], z4)
    # 2d_frame keeps frames contiguous and ascending.
    perm = oracle.morton_perm((3, 4, 4), "2d_frame")[0]
    assert np.array_equal(perm // 16, np.repeat(np.arange(3), 16))
    assert np.array_equal(perm[:16], z4)


def test_morton_roll_matches_torch_roll():
    base, _ = oracle.morton_perm((3, 4, 6))
    for r in (0, 1, 17, -5, 72):
        perm, inv = oracle.morton_perm((3, 4, 6), roll=r)
        assert np.array_equal(perm, torch.roll(torch.from_numpy(base), r).numpy())
        assert np.array_equal(perm[inv], np.arange(perm.size))


def test_morton_product_matches_oracle(pkg):
    """The library's host-side Morton (bit loops) equals the oracle's (magic masks)."""
    import importlib
    mort = importlib.import_module(f"{pkg.__name__}._morton")
    for grid, curve, roll in [((21, 30, 52), "3d", 0), ((5, 6, 8), "2d_frame", 0), ((4, 7, 9), "3d", 37)]:
        perm, inv = mort._host_perm(grid, curve, roll)["cpu"]
        rp, ri = oracle.morton_perm(grid, curve, roll)
        assert np.array_equal(perm.numpy(), rp) and np.array_equal(inv.numpy(), ri)


# -------------------------------------------------------------------- bf16
def test_bf16_round_nearest_even():
    x = np.array([1.0, 1.00390625, 1.0078125, 1.01171875, -2.5, 3.0e38, 1e-40], np.float32)
    assert np.array_equal(oracle.f32_to_bf16(x), bits(torch.from_numpy(x).to(torch.bfloat16)))
    r = np.random.default_rng(0).standard_normal(10000).astype(np.float32) * 100
    assert np.array_equal(oracle.f32_to_bf16(r), bits(torch.from_numpy(r).to(torch.bfloat16)))


# ----------------------------------------------------------------- pooling
@pytest.mark.parametrize("block", [64, 128])
def test_pool_closed_form(block):
    B, T, H, D = 2, 3 * block - 11, 3, 128
    q, k, v = (randn_bf16((B, T, H, D), s) for s in (1, 2, 3))
    kc, vc, qbar, amax = oracle.pool(bits(q), bits(k), bits(v), block, want_amax=True)
    NT = oracle.num_blocks(T, block)
    assert kc.shape[1] == oracle.npad_for(NT) and not kc[:, NT:].any()
    for j in range(NT):
        lo, hi = j * block, min(T, (j + 1) * block)
        kf = k[:, lo:hi].double().mean(1).numpy()
        vf = v[:, lo:hi].double().sum(1).numpy()
        qf = q[:, lo:hi].double().mean(1).numpy()
        # one bf16 rounding of an fp32 sum: within 1 bf16 ulp (+ fp32 noise)
        assert np.allclose(oracle.bf16_to_f32(kc[:, j]), kf, rtol=2 ** -8, atol=1e-6)
        assert np.allclose(oracle.bf16_to_f32(vc[:, j]), vf, rtol=2 ** -8, atol=1e-4)
        assert np.allclose(qbar[:, :, j], qf, rtol=1e-5, atol=1e-6)
        assert np.array_equal(amax[:, j], np.abs(v[:, lo:hi].float().numpy()).max(1))


def test_pool_canonical_order_bits():
    """kc bits equal an independent numpy restatement of the 16-partial order
    (rows r = g mod 16 summed ascending, then the fixed pairwise tree)."""
    q, k, v = (randn_bf16((1, 200, 2, 128), s) for s in (4, 5, 6))
    # exponents spread over 2^-14 .. 2^6, so that fp32 sums of bf16 values round
    # and the order shows in the bits (sums of similar bf16 values are often exact)
    g = torch.Generator().manual_seed(7)
    k = (k.float() * torch.exp2(torch.randint(-14, 7, k.shape, generator=g).float())).to(torch.bfloat16)
    kc = oracle.pool(bits(q), bits(k), bits(v), 64)[0]
    x = k.float().numpy()
    f = np.float32
    for j, (lo, n) in enumerate([(0, 64), (64, 64), (128, 64), (192, 8)]):
        part = np.zeros((16, 2, 128), f)
        for r in range(64):
            val = x[0, lo + r] if r < n else np.zeros((2, 128), f)
            part[r % 16] = (part[r % 16] + val).astype(f)
        pair = [(part[2 * i] + part[2 * i + 1]).astype(f) for i in range(8)]
        quad = [(pair[2 * i] + pair[2 * i + 1]).astype(f) for i in range(4)]
        s = ((quad[0] + quad[1]).astype(f) + (quad[2] + quad[3]).astype(f)).astype(f)
        assert np.array_equal(kc[0, j], oracle.f32_to_bf16((s / f(n)).astype(f)))
        # a plausible slip, the old 4-partial order, gives other bits somewhere
        p4 = np.zeros((4, 2, 128), f)
        for r in range(n):
            p4[r & 3] = (p4[r & 3] + x[0, lo + r]).astype(f)
        s4 = ((p4[0] + p4[1]).astype(f) + (p4[2] + p4[3]).astype(f)).astype(f)
        if n == 64:
            assert not np.array_equal(s, s4)


@pytest.mark.parametrize("centre", [False, True])
def test_moments_closed_form(centre):
    B, T, H, D, block = 1, 1000, 2, 128, 64
    q, k, v = (randn_bf16((B, T, H, D), s, scale=2.0) for s in (7, 8, 9))
    kc, vc, qbar, amax = oracle.pool(bits(q), bits(k), bits(v), block, want_amax=True)
    NT = oracle.num_blocks(T, block)
    kc2, mean, var, vscale = oracle.moments(kc, NT, centre, amax)
    kf = oracle.bf16_to_f32(kc[:, :NT]).astype(np.float64)
    assert np.allclose(mean, kf.mean(1), rtol=1e-5, atol=1e-6)
    if centre:
        cen = oracle.bf16_to_f32(kc2[:, :NT]).astype(np.float64)
        assert np.allclose(cen, kf - mean[:, None].astype(np.float64), atol=2e-2)
        assert np.allclose(var, (cen ** 2).mean(1), rtol=1e-5)
        assert np.abs(cen.mean(1)).max() < 1e-2  # centred to bf16 precision
    else:
        assert np.array_equal(kc2, kc)
        assert np.allclose(var, kf.var(1), rtol=1e-4, atol=1e-7)
    amax_all = np.abs(v.float().numpy()).max(1)
    ref = np.maximum(amax_all * (np.float32(1) / np.float32(127)), np.float32(1e-8))
    assert np.array_equal(vscale, ref.astype(np.float32))


# --------------------------------------------------------------- threshold
@pytest.mark.parametrize("mode", [0, 1])
def test_threshold_closed_form(mode):
    rng = np.random.default_rng(1)
    B, H, NT, D = 1, 3, 9, 128
    qbar = rng.standard_normal((B, H, NT, D)).astype(np.float32)
    mean = rng.standard_normal((B, H, D)).astype(np.float32) * 0.1
    var = rng.random((B, H, D)).astype(np.float32)
    scale, tau = 128 ** -0.5, 1.3
    thr = oracle.threshold(qbar, mean, var, scale, tau, mode)
    c = scale * oracle.LOG2E
    q64 = qbar.astype(np.float64)
    mu = np.einsum("bhid,bhd->bhi", q64, mean) * c
    sd = np.sqrt(np.maximum(np.einsum("bhid,bhd->bhi", q64 ** 2, var) * c * c, 0) + 1e-6)
    ref = (mu + tau * sd) if mode == 0 else tau * sd
    assert np.allclose(thr, ref.transpose(0, 2, 1), rtol=1e-5, atol=1e-5)


def test_threshold_is_gaussian_tail():
    """With Gaussian keys the routed fraction off the band is the normal tail
    P(Z > tau) (/root/reference/__init__.py:437-438 quotes 16% at tau=1)."""
    rng = np.random.default_rng(2)
    NT, D, block = 512, 128, 64
    qbar = rng.standard_normal((1, 1, NT, D)).astype(np.float32)
    kc = oracle.f32_to_bf16(rng.standard_normal((1, 512, 1, D)).astype(np.float32))
    _, mean, var, _ = oracle.moments(kc, NT, False)
    for tau in (0.5, 1.0, 1.5):
        thr = oracle.threshold(qbar, mean, var, D ** -0.5, tau, 0)
        _, _, mask, scores = oracle.route(qbar, kc, thr, NT * block, block, D ** -0.5, want_scores=True)
        frac = (scores > thr.transpose(0, 2, 1)[..., None]).mean()
        assert abs(frac - 0.5 * math.erfc(tau / math.sqrt(2))) < 0.01


# ----------------------------------------------------------------- routing
def test_route_scores_closed_form():
    q, k, v = (randn_bf16((1, 700, 2, 128), s) for s in (11, 12, 13))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=0.8, want_scores=True)
    ref = oracle.route_scores(p["qbar"], p["kc"], p["scale"])
    assert np.allclose(p["scores"], ref, rtol=1e-5, atol=1e-5)
    ex = oracle.exact_matrix(p["mask"], p["NT"])
    NT = p["NT"]
    band = np.abs(np.arange(NT)[:, None] - np.arange(NT)[None, :]) <= 1
    above = p["scores"] > p["thr"].transpose(0, 2, 1)[..., None]
    assert np.array_equal(ex, above | band[None, None])
    # lists: ascending, counts agree with the mask
    for h in range(2):
        for i in range(NT):
            n = p["counts"][0, h, i]
            assert n == ex[0, h, i].sum()
            assert np.array_equal(p["lists"][0, h, i, :n], np.nonzero(ex[0, h, i])[0])


def test_route_sinks_and_band():
    q, k, v = (randn_bf16((1, 1280, 1, 128), s) for s in (14, 15, 16))
    NT = 20
    p = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=1e30, sink_kv=(0, 3), sink_q=(5, 7))
    ex = oracle.exact_matrix(p["mask"], NT)[0, 0]
    for i in range(NT):
        if 5 <= i < 7:
            assert ex[i].all()  # dense query rows
        else:
            want = {j for j in range(NT) if abs(i - j) <= 1 or j < 3}
            assert set(np.nonzero(ex[i])[0]) == want
    p = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=-1e30)
    assert oracle.exact_matrix(p["mask"], NT).all()


def test_tie_band_helper():
    s = np.zeros((1, 1, 2, 2), np.float32)
    thr = np.zeros((1, 2, 1), np.float32)
    a = np.array([[[[True, False], [False, True]]]])
    b = a.copy()
    assert oracle.tie_count(s, thr, a, b) == (0, True)
    b[0, 0, 0, 1] = True
    assert oracle.tie_count(s, thr, a, b) == (1, True)
    s[0, 0, 0, 1] = 1.0
    assert oracle.tie_count(s, thr, a, b) == (1, False)


# ------------------------------------------------------------------- quant
def test_quant_known_answers():
    D = 128
    x = np.zeros((1, 4, 1, D), np.float32)
    x[0, 0, 0, :4] = [127.0, -127.0, 0.5, -0.5]      # scale 1: ties round away from zero
    x[0, 1, 0, 0] = 2.0                                # scale 2/127: max -> 127
    x[0, 1, 0, 1] = -2.0                               # never -128
    x[0, 1, 0, 2] = 1.0 / 127.0                        # rounds to 0 or +1 consistently
    x[0, 3, 0, :] = 3.0                                 # constant row -> all 127
    xi, xs = oracle.quant_rows(oracle.f32_to_bf16(x))
    assert xs[0, 0, 0] == np.float32(1.0)
    assert list(xi[0, 0, 0, :4]) == [127, -127, 1, -1]
    assert xi[0, 1, 0, 0] == 127 and xi[0, 1, 0, 1] == -127
    assert xs[0, 2, 0] == np.float32(1e-8) and not xi[0, 2].any()  # zero row: floor scale
    assert (xi[0, 3] == 127).all()
    assert xi.min() >= -127


def test_quant_blocked_known_answers():
    """Per-128-token-block scales (BASELINE config 3's variant): one scale per
    (batch, block, head) from the block's |max|, the per-token code rule, the
    scale written for every token of the block; a ragged last block has its
    own scale."""
    D, QB = 128, 128
    x = np.zeros((1, 200, 2, D), np.float32)
    x[0, 5, 0, 3] = 127.0                               # block 0, head 0: scale 1
    x[0, 9, 0, :4] = [2.5, -2.5, 1.25, -0.5]           # ties away from zero at scale 1
    x[0, 130, 0, 7] = -63.5                             # block 1 (72 tokens): scale 0.5
    x[0, 131, 0, :2] = [1.25, -0.25]                    # -> 2.5 -> 3, -0.5 -> -1
    x[0, :, 1, :] = 3.0                                 # head 1: constant -> all 127
    xi, xs = oracle.quant_rows(oracle.f32_to_bf16(x), block=QB)
    assert (xs[0, :128, 0] == np.float32(1.0)).all() and (xs[0, 128:, 0] == np.float32(0.5)).all()
    assert list(xi[0, 9, 0, :4]) == [3, -3, 1, -1]
    assert xi[0, 5, 0, 3] == 127 and xi[0, 130, 0, 7] == -127
    assert list(xi[0, 131, 0, :2]) == [3, -1]
    assert (xi[0, :, 1] == 127).all() and (xs[0, :, 1] == np.float32(3.0 / 127.0)).all()


def test_quant_blocked_equals_per_token_on_equal_row_maxima():
    """The blocked scale is the largest per-token scale of its block (fl(a/127)
    is monotonic), smoothing included; and when every token row of a block
    holds the block's |max| the per-block and per-token rules give the same
    codes and scales."""
    rng = np.random.default_rng(11)
    x = rng.standard_normal((2, 300, 3, 128)).astype(np.float32)
    mean = (rng.standard_normal((2, 3, 128)) * 0.1).astype(np.float32)
    xb = oracle.f32_to_bf16(x)
    ts = oracle.quant_rows(xb, mean)[1]
    bs = oracle.quant_rows(xb, mean, block=128)[1]
    for j in range(0, 300, 128):
        blk = slice(j, min(j + 128, 300))
        assert np.all(bs[:, blk] == ts[:, blk].max(1, keepdims=True))
    xr = oracle.bf16_to_f32(xb)                          # plant each block's |max| in every row
    for j in range(0, 300, 128):
        blk = slice(j, min(j + 128, 300))
        xr[:, blk, :, 0] = np.abs(xr[:, blk]).max(axis=(1, 3))[:, None, :]
    xp = oracle.f32_to_bf16(xr)                          # bf16 values: exact
    ti, ts = oracle.quant_rows(xp)
    bi, bs = oracle.quant_rows(xp, block=128)
    assert np.array_equal(bi, ti) and np.array_equal(bs, ts)


def test_division_free_scale_matches_ieee():
    """The quantisers' per-token scale fl(amax / 127) computed without a
    division (one fma residual step on amax * fl(1/127)) equals the IEEE
    quotient: every float in the binades that hold realistic row maxima, and a
    stride-97 sweep of all non-negative finite floats. (An exhaustive sweep of
    all 2^31 was run once; it takes ~40 s.)"""
    import ctypes
    L = oracle.lib()
    f = L.or_div127_mismatches
    f.argtypes = [ctypes.c_uint32] * 3
    f.restype = ctypes.c_uint64
    assert f(0x3c000000, 0x42000000, 1) == 0   # [2^-7, 32): every float
    assert f(0, 0x7f800000, 97) == 0            # the whole range, strided
    assert f(0, 1 << 23, 1) == 0                # denormals


def test_biased_code_fast_path_matches_contract():
    """The quantisers' fast path: with rr within 1 ulp of 1/s (v_rcp_f32),
    v = fl(fl(x * rr) + 128) and v farther than 4e-5 from every half-integer,
    rint(v) - 128 is the contract's code trunc(fl(q + copysign(0.5, q))) of the
    IEEE quotient q = fl(x / s). Random rows at their own scales, plus values
    placed on and around half-integer quotients (the cases the guard sends to
    the division path); rr at RN(1/s) and one ulp either side."""
    rng = np.random.default_rng(11)
    f32 = np.float32
    n = 400_000
    amax = (10.0 ** rng.uniform(-7, 2, n)).astype(f32)
    s = np.maximum(amax / f32(127), f32(1e-8)).astype(f32)
    # quotients uniform in [-127, 127], and clustered near k + 1/2
    k = rng.integers(-127, 127, n).astype(np.float64)
    target = np.where(rng.random(n) < 0.5, rng.uniform(-127, 127, n),
                      k + 0.5 + rng.normal(0, 3e-5, n))
    target = np.clip(target, -127, 127)
    x = oracle.bf16_to_f32(oracle.f32_to_bf16((target * s).astype(f32)))
    x = np.where(np.abs(x) <= f32(127) * s, x, np.sign(x) * f32(127) * s).astype(f32)
    q = (x / s).astype(f32)
    t = (q + np.copysign(f32(0.5), q)).astype(f32)
    want = np.clip(np.trunc(t), -127, 127)
    r0 = (f32(1) / s).astype(f32)
    taken = 0
    for rr in (np.nextafter(r0, f32(0)), r0, np.nextafter(r0, f32(np.inf))):
        v = ((x * rr).astype(f32) + f32(128)).astype(f32)
        fast = np.abs(v - np.rint(v)) < f32(0.5) - f32(4e-5)
        got = np.rint(v) - 128
        assert np.array_equal(got[fast], want[fast])
        assert np.all(np.abs(got[fast]) <= 127)
        taken += int(fast.sum())
    assert taken > 2 * n       # most values take the fast path


def test_quant_smoothing_and_v():
    x = randn_bf16((2, 50, 3, 128), 17, scale=4.0)
    mean = np.random.default_rng(3).standard_normal((2, 3, 128)).astype(np.float32)
    xi, xs = oracle.quant_rows(bits(x), mean)
    y = x.float().numpy() - mean[:, None]
    s = np.maximum(np.abs(y).max(-1) / np.float32(127), np.float32(1e-8))
    assert np.array_equal(xs, s.astype(np.float32))
    deq = xi.astype(np.float64) * xs[..., None]
    assert np.abs(deq - y).max() <= 0.5 * xs.max() * (1 + 1e-5)
    vs = np.maximum(np.abs(x.float().numpy()).max(1) / np.float32(127), np.float32(1e-8)).astype(np.float32)
    vi = oracle.quant_v(bits(x), vs)
    assert np.abs(vi.astype(np.float64) * vs[:, None] - x.float().numpy()).max() <= 0.5 * vs.max() * (1 + 1e-5)


# ----------------------------------------------------------------- forward
def _rows(prep, B, H):
    return [(b, h, i) for b in range(B) for h in range(H) for i in range(prep["NT"])]


@pytest.mark.parametrize("block,tau", [(64, 0.9), (128, 0.5), (64, 1.5)])
def test_forward_port_vs_closed_form(block, tau):
    B, T, H = 1, 2 * block + 37 + 5 * block, 2
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (21, 22, 23))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=block, tau=tau)
    rows = _rows(p, B, H)
    cf = oracle.forward_closed_form(bits(q), bits(k), bits(v), p, rows)
    exact = oracle.forward_port(bits(q), bits(k), bits(v), p, rows, round_p=False)
    port = oracle.forward_port(bits(q), bits(k), bits(v), p, rows)
    for r in rows:
        assert np.abs(exact[r] - cf[r]).max() < 1e-5     # the algebra
        assert np.abs(port[r] - cf[r]).max() < 5e-3      # + bf16 rounding of P
    # The pooled term matters: dropping it (dense SDPA over the exact blocks only)
    # is a different function.
    dm = oracle.forward_dense_block_mask(bits(q), bits(k), bits(v), p, rows)
    assert max(np.abs(dm[r] - cf[r]).max() for r in rows) > 1e-3


def test_forward_all_exact_is_dense_sdpa():
    B, T, H = 1, 300, 2
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (24, 25, 26))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=-1e30)
    rows = _rows(p, B, H)
    port = oracle.forward_port(bits(q), bits(k), bits(v), p, rows, round_p=False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(t.double().transpose(1, 2) for t in (q, k, v))).transpose(1, 2).numpy()
    for (b, h, i), o in port.items():
        assert np.abs(o - ref[b, i * 64:i * 64 + o.shape[0], h]).max() < 1e-5


def test_forward_blockwise_constant_kv_is_exact():
    """K and V constant inside every block: the pooled key/value are exact, so the
    output is dense SDPA for any routing."""
    B, H, block = 1, 2, 64
    T = 5 * block
    rng = np.random.default_rng(4)
    kb = rng.integers(-3, 4, size=(B, 5, H, 128)) / 4.0   # few mantissa bits: sums exact
    vb = rng.integers(-3, 4, size=(B, 5, H, 128)) / 4.0
    k = torch.from_numpy(np.repeat(kb, block, axis=1)).to(torch.bfloat16)
    v = torch.from_numpy(np.repeat(vb, block, axis=1)).to(torch.bfloat16)
    q = randn_bf16((B, T, H, 128), 27)
    p = oracle.prepare(bits(q), bits(k), bits(v), block=block, tau=1.0)
    assert not oracle.exact_matrix(p["mask"], 5).all()  # some blocks are pooled
    rows = _rows(p, B, H)
    port = oracle.forward_port(bits(q), bits(k), bits(v), p, rows, round_p=False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(t.double().transpose(1, 2) for t in (q, k, v))).transpose(1, 2).numpy()
    for (b, h, i), o in port.items():
        assert np.abs(o - ref[b, i * block:(i + 1) * block, h]).max() < 1e-5


def test_forward_sink_rows_are_dense():
    B, T, H = 1, 640, 1
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (28, 29, 30))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=2.0, sink_q=(2, 4))
    port = oracle.forward_port(bits(q), bits(k), bits(v), p, [(0, 0, 2), (0, 0, 3)], round_p=False)
    ref = torch.nn.functional.scaled_dot_product_attention(
        *(t.double().transpose(1, 2) for t in (q, k, v))).transpose(1, 2).numpy()
    assert np.abs(port[(0, 0, 2)] - ref[0, 128:192, 0]).max() < 1e-5
    assert np.abs(port[(0, 0, 3)] - ref[0, 192:256, 0]).max() < 1e-5


def test_forward_morton_neutral_when_dense():
    """attn(perm x) = perm attn(x) with every block exact."""
    grid = (2, 4, 8)
    B, H, T = 1, 1, 64
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (31, 32, 33))
    perm, inv = oracle.morton_perm(grid)
    p0 = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=-1e30)
    qp, kp, vp = (t[:, perm] for t in (q, k, v))
    p1 = oracle.prepare(bits(qp), bits(kp), bits(vp), block=64, tau=-1e30)
    o0 = oracle.forward_port(bits(q), bits(k), bits(v), p0, [(0, 0, 0)], round_p=False)[(0, 0, 0)]
    o1 = oracle.forward_port(bits(qp), bits(kp), bits(vp), p1, [(0, 0, 0)], round_p=False)[(0, 0, 0)]
    assert np.abs(o1[inv] - o0).max() < 1e-5


@pytest.mark.parametrize("int8_pv", [False, True])
def test_forward_int8_port_vs_closed_form(int8_pv):
    B, T, H, block = 1, 600, 2, 64
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (34, 35, 36))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=block, tau=0.7, int8=True, int8_pv=int8_pv)
    rows = _rows(p, B, H)
    qd = p["qi"].astype(np.float64) * p["qs"][..., None]
    kd = p["ki"].astype(np.float64) * p["ks"][..., None]
    # centred K: the closed form uses the smoothed keys for the exact branch
    # (a per-row constant shift of the scores cancels in the softmax)
    cf = oracle.forward_closed_form(bits(q), bits(k), bits(v), p, rows, qk=(qd, kd))
    port = oracle.forward_int8_port(bits(q), bits(v), p, rows, int8_pv=int8_pv)
    got = np.concatenate([port[r].ravel() for r in rows])
    ref = np.concatenate([cf[r].ravel() for r in rows])
    assert cosine(got, ref) > (0.999 if int8_pv else 0.9999)


@pytest.mark.parametrize("block,T", [(64, 600), (128, 700), (128, 2 * 128 + 100)])
def test_forward_int8_kernel_codes_constant_v_is_exact(block, T):
    """The kernel-arithmetic INT8 variant normalises by the sum of the codes it
    multiplies, so with V the same vector on every token the output is exactly
    that vector (weights sum to one); the reference arithmetic (fp32 pe sums,
    trunc(pe*127+0.5) codes) is off by the quantisation of P. Every block is
    exact here (the pooled branch rounds P to bf16 in both arithmetics). Covers
    the block-128 ragged last block of more than 64 keys (T = 356) that the
    kernel quantises per 64-key tile."""
    B, H = 1, 2
    q, k = (randn_bf16((B, T, H, 128), s) for s in (50, 51))
    row = torch.linspace(-2, 2, 128).to(torch.bfloat16)
    v = row.expand(B, T, H, 128).contiguous()
    p = oracle.prepare(bits(q), bits(k), bits(v), block=block, tau=-1e30, int8=True, int8_pv=True)
    rows = _rows(p, B, H)
    want = row.float().numpy()
    ker = oracle.forward_int8_port(bits(q), bits(v), p, rows, int8_pv=True, codes="kernel")
    ref = oracle.forward_int8_port(bits(q), bits(v), p, rows, int8_pv=True, codes="reference")
    ker_err = max(np.abs(ker[r] - want).max() for r in rows)
    ref_err = max(np.abs(ref[r] - want).max() for r in rows)
    assert ker_err < 2e-6, ker_err
    assert ref_err > 50 * ker_err


def test_forward_int8_kernel_codes_track_reference_per_block():
    """Both INT8 arithmetics agree per query block to the INT8 tolerance, and
    coincide wherever every code is 127 (all scores of a block equal)."""
    B, T, H, block = 1, 1000, 2, 64
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (52, 53, 54))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=block, tau=0.7, int8=True, int8_pv=True)
    rows = _rows(p, B, H)
    ker = oracle.forward_int8_port(bits(q), bits(v), p, rows, codes="kernel")
    ref = oracle.forward_int8_port(bits(q), bits(v), p, rows, codes="reference")
    assert min(cosine(ker[r], ref[r]) for r in rows) > 0.999
    # identical keys within every block: pe = 1, both codes 127, same sums
    kb = k.clone()
    for j in range(0, T, block):
        kb[:, j:j + block] = k[:, j:j + 1]
    p2 = oracle.prepare(bits(q), bits(kb), bits(v), block=block, tau=0.7, int8=True, int8_pv=True)
    ker2 = oracle.forward_int8_port(bits(q), bits(v), p2, rows, codes="kernel")
    ref2 = oracle.forward_int8_port(bits(q), bits(v), p2, rows, codes="reference")
    assert max(np.abs(ker2[r] - ref2[r]).max() for r in rows) < 1e-5


def _hand_prep(T, block, qs_val, ki0, ks_val, vi0, vscale0=1.0):
    """A one-head INT8 prep by hand: every block exact for every query block;
    query rows carry qi[:, 0] = 1 (scale qs_val), key t carries ki[t, 0] =
    ki0[t] with scale ks_val and vi[t, 0] = vi0[t]; other channels zero.
    scale = ln 2, so the log2-domain score of key t is ki0[t] * qs_val * ks_val."""
    NT = -(-T // block)
    W = -(-NT // 32)
    mask = np.zeros((1, 1, NT, W), np.uint32)
    for j in range(NT):
        mask[..., j >> 5] |= np.uint32(1) << np.uint32(j & 31)
    qi = np.zeros((1, T, 1, 128), np.int8)
    qi[..., 0] = 1
    ki = np.zeros((1, T, 1, 128), np.int8)
    ki[0, :, 0, 0] = ki0
    vi = np.zeros((1, T, 1, 128), np.int8)
    vi[0, :, 0, 0] = vi0
    vscale = np.zeros((1, 1, 128), np.float32)
    vscale[..., 0] = vscale0
    npad = -(-NT // 64) * 64
    kc = np.zeros((1, npad, 1, 128), np.uint16)  # pooled keys/values: unused (nothing approximate)
    return dict(block=block, T=T, NT=NT, scale=float(np.float32(math.log(2.0))), mask=mask, qi=qi,
                kc=kc, vc=kc,
                qs=np.full((1, T, 1), qs_val, np.float32), ki=ki,
                ks=np.full((1, T, 1), ks_val, np.float32), vi=vi, vscale=vscale)


def test_forward_int8_running_known_answer():
    """Running-max codes by hand (block 64, two exact blocks, log2 scores
    ki/8): block 0 has one key at 2.5 and 63 at 0, so m = ceil(2.5) = 3, codes
    rint(127 * 2^-0.5) = 90 and rint(127 / 8) = 16; block 1 has one key at 4.25
    and 63 at 0, so m = 5: the int32 sums shift right by 2 (floor) and the
    code sum scales by 1/4 (exact) before codes rint(127 * 2^-0.75) = 76 and
    rint(127 / 32) = 4 add. With v codes 100 / 1 in block 0 and -50 / 2 in
    block 1: sums 90*100 + 63*16 = 10008, code sum 1098; then 2502 and 274.5;
    + 76*(-50) + 63*4*2 = -3296 and + 76 + 252: -794 and 602.5; output
    -794 / 602.5 on channel 0."""
    T, block = 128, 64
    ki0 = np.zeros(T, np.int64)
    ki0[0], ki0[64] = 20, 34
    vi0 = np.array([100] + [1] * 63 + [-50] + [2] * 63)
    prep = _hand_prep(T, block, 1.0, ki0, 0.125, vi0)
    q = np.zeros((1, T, 1, 128), np.uint16)  # the pooled branch is empty: every block exact
    out = oracle.forward_int8_port(q, q, prep, [(0, 0, 0)], codes="running")[(0, 0, 0)]
    assert np.allclose(out[:, 0], -794.0 / 602.5, rtol=1e-6, atol=0)
    assert np.all(out[:, 1:] == 0)
    # the block-max arithmetics give other values (codes 127 at each block's max)
    ker = oracle.forward_int8_port(q, q, prep, [(0, 0, 0)], codes="kernel")[(0, 0, 0)]
    assert abs(float(ker[0, 0]) - (-794.0 / 602.5)) > 1e-2


def test_forward_int8_running_headroom_rise():
    """The running max rises by one more when a lane's half of a row's code
    sum passes 2^23 (the int32 sums' headroom): 2070 blocks of 64 keys, every
    score 0, so m = 0 and every code is 127; each block adds 32 * 127 = 4064
    to each half (keys k mod 8 < 4 and the rest), which passes 2^23 after 2065
    blocks (8392160), so block 2066 raises m to 1: sums >> 1, code sum halved,
    codes rint(63.5) = 64 (half to even). v codes 1 in the first 2065 blocks,
    3 in the last five: sums 2065*64*127 = 16784320 -> 8392160 + 5*64*64*3 =
    8453600, code sum 8392160 + 5*64*64 = 8412640."""
    T, block = 2070 * 64, 64
    vi0 = np.where(np.arange(T) < 2065 * 64, 1, 3)
    prep = _hand_prep(T, block, 1.0, np.zeros(T, np.int64), 1.0, vi0)
    q = np.zeros((1, T, 1, 128), np.uint16)
    out = oracle.forward_int8_port(q, q, prep, [(0, 0, 0)], codes="running")[(0, 0, 0)]
    assert np.allclose(out[:, 0], 8453600.0 / 8412640.0, rtol=1e-7, atol=0)
    no_rise = (16784320 + 5 * 64 * 127 * 3) / (16784320 + 5 * 64 * 127)
    assert abs(float(out[0, 0]) - no_rise) > 1e-5


@pytest.mark.parametrize("block", [64, 128])
def test_forward_int8_running_tracks_reference_per_block(block):
    """The running-max arithmetic against the reference's per query block
    (north_star's INT8 tolerance), on Gaussian inputs -- the hard case for
    codes against the running max: the blocks' maxima spread, so blocks below
    the running max get coarse codes (measured worst 0.9992-0.9993) -- with a
    ragged last block (T % block != 0)."""
    B, T, H = 1, 3000, 2
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (55, 56, 57))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=block, tau=0.9, int8=True, int8_pv=True)
    rows = _rows(p, B, H)
    run = oracle.forward_int8_port(bits(q), bits(v), p, rows, codes="running")
    ref = oracle.forward_int8_port(bits(q), bits(v), p, rows, codes="reference")
    assert min(cosine(run[r], ref[r]) for r in rows) >= 0.999


def test_cfg0_plumbing_d64():
    """BASELINE config 0 (B1 H4 D64, 4x32x32 grid -> N 4096, block 64, tau 0.9,
    smooth field + 0.3 noise, Morton 3d) through the CPU path: the Morton
    permutation against the brute-force bit loop, routing against the float64
    closed form of the scores (decisions may differ only inside the tie band),
    and the masked torch path and the reference loop against the float64
    augmented-key closed form. Inputs are rounded to bf16, the kernels'
    arithmetic type."""
    import bench
    cfg = bench.CONFIGS[0]
    q, k, v = bench.make_inputs(cfg, "cpu", dtype=torch.float32)
    perm, inv = oracle.morton_perm(cfg["grid"], "3d")
    assert np.array_equal(perm, _brute_perm(cfg["grid"], "3d"))
    assert np.array_equal(perm[inv], np.arange(perm.size))
    q, k, v = (t[:, perm].to(torch.bfloat16) for t in (q, k, v))
    B, T, H, D = q.shape
    assert (B, T, H, D) == (1, 4096, 4, 64)
    p = oracle.prepare(bits(q), bits(k), bits(v), block=cfg["block"], tau=cfg["tau"],
                       want_scores=True)
    NT = p["NT"]
    R = oracle.route_scores(p["qbar"], p["kc"], p["scale"])
    thr = np.transpose(p["thr"], (0, 2, 1))[..., None].astype(np.float64)
    i, j = np.meshgrid(np.arange(NT), np.arange(NT), indexing="ij")
    want = (R > thr) | (np.abs(i - j) <= 1)
    got = oracle.exact_matrix(p["mask"], NT)
    n_diff, in_band = oracle.tie_count(p["scores"], p["thr"], got, want)
    assert in_band and n_diff <= 4
    density = got.mean()
    assert 0.05 < density < 0.6
    rows = [(0, h, ii) for h in range(H) for ii in range(0, NT, 7)]
    cf = oracle.forward_closed_form(bits(q), bits(k), bits(v), p, rows)
    mt = oracle.masked_attention_torch(q.float(), k.float(), v.float(), p, heads=list(range(H)),
                                       qblocks=list(range(0, NT, 7)))
    port = oracle.forward_port(bits(q), bits(k), bits(v), p, rows)
    for r in rows:
        assert np.abs(mt[r].numpy() - cf[r]).max() < 1e-5
        assert np.abs(port[r] - cf[r]).max() < 2e-2
        assert cosine(port[r], cf[r]) > 0.9995


def test_masked_attention_torch_matches_closed_form():
    B, T, H = 1, 333, 2
    q, k, v = (randn_bf16((B, T, H, 128), s) for s in (37, 38, 39))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=0.6)
    rows = _rows(p, B, H)
    cf = oracle.forward_closed_form(bits(q), bits(k), bits(v), p, rows)
    mt = oracle.masked_attention_torch(q.float(), k.float(), v.float(), p)
    for r in rows:
        assert np.abs(mt[r].numpy() - cf[r]).max() < 1e-5


def test_routed_flops_counts_valid_tokens():
    q, k, v = (randn_bf16((1, 300, 1, 128), s) for s in (40, 41, 42))
    p = oracle.prepare(bits(q), bits(k), bits(v), block=128, tau=-1e30)
    # all exact: 4*D*sum_i len_i*T = 4*D*T^2
    assert oracle.routed_flops(p["mask"], 300, 128, 128, mask=True) == 4 * 128 * 300 * 300
