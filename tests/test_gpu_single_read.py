"""The single-read INT8 preparation (solattn_prep_int8) through the C ABI: every
output -- pooled keys and values, centroids, centred kc, its moments, the V
scale, the Q / K / V codes and scales -- bit for bit against the two-pass entry
points (solattn_pool, solattn_moments, solattn_quant_rows, solattn_quant_v) and
against the oracle, with the barrier's bound flag left clear; shapes that do
not fit two heads on the device are refused with SOLATTN_EUNSUPPORTED and the
Python API falls back to the two passes.
Reference: /root/reference/_fused_prep.py:62-98 (two reads of K and V)."""

import importlib

import numpy as np
import pytest
import torch

import oracle
from _util import bits, randn_bf16

pytestmark = pytest.mark.gpu

CASES = [  # (B, T, H, block): ragged tails, one-block spans, many heads
    (2, 777, 3, 128), (1, 1000, 2, 64), (1, 4096, 24, 64), (1, 129, 5, 128), (3, 64, 4, 64),
    (1, 2500, 8, 128)]


def _mods(pkg):
    n = pkg.__name__
    return (importlib.import_module(f"{n}._capi"), importlib.import_module(f"{n}._preprocess"),
            importlib.import_module(f"{n}._fused_prep"))


def _alloc(B, T, H, block, int8_pv, dev):
    NT = -(-T // block)
    npad = -(-NT // 64) * 64
    f32 = dict(device=dev, dtype=torch.float32)
    out = dict(kc=torch.zeros((B, npad, H, 128), device=dev, dtype=torch.bfloat16),
               qbar=torch.empty((B, H, NT, 128), **f32), kc_mean=torch.empty((B, H, 128), **f32),
               kc_var=torch.empty((B, H, 128), **f32),
               qi=torch.empty((B, T, H, 128), device=dev, dtype=torch.int8),
               qs=torch.empty((B, T, H), **f32), ks=torch.empty((B, T, H), **f32))
    out["vc"] = torch.zeros_like(out["kc"])
    out["ki"] = torch.empty_like(out["qi"])
    if int8_pv:
        out.update(vamax=torch.empty((B, NT, H, 128), **f32), vscale=torch.empty((B, H, 128), **f32),
                   vi=torch.empty_like(out["qi"]))
    return out, NT, npad


def _strides(t):
    return t.stride(0), t.stride(1), t.stride(2)


def _single_read(capi, q, k, v, block, int8_pv):
    B, T, H, D = q.shape
    o, NT, npad = _alloc(B, T, H, block, int8_pv, q.device)
    sync = torch.full((capi.LIB.solattn_prep_int8_sync_bytes(B, H),), 0xAB, device=q.device,
                      dtype=torch.uint8)  # garbage: the call resets it
    p = capi.ptr
    rc = capi.LIB.solattn_prep_int8(
        p(q), *_strides(q), p(k), *_strides(k), p(v), *_strides(v), B, T, H, D, block, p(o["kc"]),
        p(o["vc"]), npad, p(o["qbar"]), p(o["kc_mean"]), p(o["kc_var"]), p(o.get("vamax")),
        p(o.get("vscale")), p(o["qi"]), p(o["qs"]), p(o["ki"]), p(o["ks"]), 0, p(o.get("vi")), T,
        p(sync), sync.numel(), capi.stream(q.device))
    torch.cuda.synchronize()
    return rc, o, sync


def _two_pass(capi, q, k, v, block, int8_pv):
    B, T, H, D = q.shape
    o, NT, npad = _alloc(B, T, H, block, int8_pv, q.device)
    p, s = capi.ptr, capi.stream(q.device)
    capi.call("solattn_pool", p(q), *_strides(q), p(k), *_strides(k), p(v), *_strides(v), B, T, H,
              D, block, p(o["kc"]), p(o["vc"]), npad, p(o["qbar"]), p(o.get("vamax")), s)
    capi.call("solattn_moments", p(o["kc"]), npad, B, NT, H, D, 1, p(o["kc_mean"]),
              p(o["kc_var"]), p(o.get("vamax")), p(o.get("vscale")), s)
    capi.call("solattn_quant_rows", p(q), *_strides(q), B, T, H, D, None, p(o["qi"]), p(o["qs"]),
              T, s)
    capi.call("solattn_quant_rows", p(k), *_strides(k), B, T, H, D, p(o["kc_mean"]), p(o["ki"]),
              p(o["ks"]), T, s)
    if int8_pv:
        capi.call("solattn_quant_v", p(v), *_strides(v), B, T, H, D, p(o["vscale"]), p(o["vi"]),
                  T, s)
    torch.cuda.synchronize()
    return o


def _u(t):
    x = t.detach().cpu()
    if x.dtype == torch.bfloat16:
        return x.view(torch.int16).numpy()
    if x.dtype == torch.float32:
        return x.numpy().view(np.uint32)
    return x.numpy()


@pytest.mark.parametrize("int8_pv", [True, False])
@pytest.mark.parametrize("case", CASES)
def test_single_read_matches_two_pass_and_oracle(pkg, dev, case, int8_pv):
    capi = _mods(pkg)[0]
    B, T, H, block = case
    print(f"[single read] case={case} int8_pv={int8_pv}", flush=True)
    q, k, v = (randn_bf16((B, T, H, 128), s, scale=sc) for s, sc in ((30, 1.0), (31, 2.0), (32, 0.7)))
    k = k + randn_bf16((1, 1, H, 128), 33)  # a per-head key offset: the smoothing matters
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    rc, one, sync = _single_read(capi, qd, kd, vd, block, int8_pv)
    if rc == -2:
        pytest.skip(f"shape does not fit two heads on this device: "
                    f"{capi.LIB.solattn_last_error().decode()}")
    assert rc == 0, capi.LIB.solattn_last_error()
    assert int(sync[:4].cpu().view(torch.int32)[0]) == 0  # every barrier met in time
    two = _two_pass(capi, qd, kd, vd, block, int8_pv)
    NT = -(-T // block)
    for name in one:
        a, b = _u(one[name]), _u(two[name])
        if name in ("kc", "vc"):
            a, b = a[:, :NT], b[:, :NT]
        assert np.array_equal(a, b), name
    ref = oracle.prepare(bits(q), bits(k), bits(v), block=block, tau=0.9, int8=True,
                         int8_pv=int8_pv)
    assert np.array_equal(_u(one["kc"])[:, :NT].view(np.uint16), ref["kc"][:, :NT])
    assert np.array_equal(_u(one["vc"])[:, :NT].view(np.uint16), ref["vc"][:, :NT])
    for name in ("qbar", "kc_mean", "kc_var"):
        assert np.array_equal(_u(one[name]), ref[name].view(np.uint32)), name
    for name in ("qi", "ki"):
        assert np.array_equal(_u(one[name]), ref[name][:, :T]), name
    for name in ("qs", "ks"):
        assert np.array_equal(_u(one[name]), ref[name][:, :T].view(np.uint32)), name
    if int8_pv:
        assert np.array_equal(_u(one["vi"]), ref["vi"][:, :T])
        assert np.array_equal(_u(one["vscale"]), ref["vscale"].view(np.uint32))
        assert np.array_equal(_u(one["vamax"]), ref["vamax_part"].view(np.uint32))


def test_single_read_refuses_one_head_and_python_falls_back(pkg, dev):
    """B*H = 1 leaves one team: refused with SOLATTN_EUNSUPPORTED (no launch);
    fused_preprocess_routing then runs the two passes, same bits as the oracle."""
    capi, _, fp = _mods(pkg)
    q, k, v = (randn_bf16((1, 1000, 1, 128), s) for s in (40, 41, 42))
    qd, kd, vd = (t.to(dev) for t in (q, k, v))
    rc, _, _ = _single_read(capi, qd, kd, vd, 64, True)
    assert rc == -2 and b"single-read" in capi.LIB.solattn_last_error()
    r, qi, qs, ki, ks, vi = fp.fused_preprocess_routing(qd, kd, vd, tau=0.9, scale=128 ** -0.5,
                                                        block=64)
    ref = oracle.prepare(bits(q), bits(k), bits(v), block=64, tau=0.9, int8=True)
    assert np.array_equal(ki.cpu().numpy(), ref["ki"]) and np.array_equal(vi.cpu().numpy(), ref["vi"])
    assert np.array_equal(r.counts.cpu().numpy(), ref["counts"])


def test_python_single_read_option_same_bits(pkg, dev):
    """fused_preprocess_routing(single_read=True) hands the forward the same
    routing, codes and scales as the default two passes."""
    _, _, fp = _mods(pkg)
    q, k, v = (randn_bf16((1, 1500, 6, 128), s).to(dev) for s in (50, 51, 52))
    a = fp.fused_preprocess_routing(q, k, v, tau=0.8, scale=128 ** -0.5, block=128)
    b = fp.fused_preprocess_routing(q, k, v, tau=0.8, scale=128 ** -0.5, block=128,
                                    single_read=True)
    ra, rb = a[0], b[0]
    for name in ("kc", "vc", "threshold", "qbar", "kc_mean", "kc_var", "counts", "mask", "vscale"):
        assert torch.equal(getattr(ra, name), getattr(rb, name)), name
    for x, y, name in zip(a[1:], b[1:], ("qi", "qs", "ki", "ks", "vi")):
        assert torch.equal(x, y), name
