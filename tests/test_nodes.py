"""The ComfyUI boundary on the CPU, with a stand-in comfy package: block/tau
parsing, every gate of the override, chaining, the exception -> dense
fallback, stats, layout adaptation, the sink rule and the node's execute."""

import importlib

import pytest
import torch


@pytest.fixture
def disp(pkg):
    d = importlib.import_module(f"{pkg.__name__}._dispatch")
    d.reset_sol_attn_stats()
    return d


def test_node_layer_registered(pkg):
    from comfy.ldm.modules import attention

    assert hasattr(pkg, "SolAttnPatch") and hasattr(pkg, "SolAttnBlockProbe")
    assert attention.REGISTERED.get("sol_attn") is pkg.attention_sol
    schema = pkg.SolAttnPatch.define_schema()
    names = [i.name for i in schema.inputs]
    for name in ("model", "tau", "start_percent", "end_percent", "min_tokens", "int8_qk",
                 "sink_conditioning", "morton", "morton_curve", "int8_pv", "verbose", "use_tma",
                 "tau_profile", "dense_blocks", "block_size", "int8_pv_codes"):
        assert name in names
    assert schema.node_id == "SolAttnPatch"


def test_parse_blocks(disp):
    assert disp.parse_blocks("0-3,47,-1", 50) == frozenset({0, 1, 2, 3, 47, 49})
    assert disp.parse_blocks(" 5 - 2 , ", 10) == frozenset({2, 3, 4, 5})
    assert disp.parse_blocks("-2--1", 10) == frozenset({8, 9})
    assert disp.parse_blocks("", 10) == frozenset()
    assert disp.parse_blocks("8-20", 10) == frozenset({8, 9})
    with pytest.raises(ValueError):
        disp.parse_blocks("a-b", 10)


def test_parse_tau_profile(disp):
    prof = disp.parse_tau_profile("0-2=2.0; 1=0.5\n# comment\n-1=1.1  # tail", 10)
    assert prof == {0: 2.0, 1: 0.5, 2: 2.0, 9: 1.1}
    with pytest.raises(ValueError):
        disp.parse_tau_profile("3", 10)
    with pytest.raises(ValueError):
        disp.parse_tau_profile("3=x", 10)


def test_sink_blocks(disp):
    opts = {"sol_h3_video_span": (100, 1000)}
    assert disp._sink_blocks(opts, 1000, "exact_kv", 64) == ((0, 2), (0, 0))
    assert disp._sink_blocks(opts, 1000, "exact_kv_and_rows", 64) == ((0, 2), (0, 2))
    assert disp._sink_blocks(opts, 1000, "exact_kv", 128) == ((0, 1), (0, 0))
    assert disp._sink_blocks(opts, 999, "exact_kv", 64) == ((0, 0), (0, 0))
    assert disp._sink_blocks(opts, 1000, "off", 64) == ((0, 0), (0, 0))
    assert disp._sink_blocks({}, 1000, "exact_kv", 64) == ((0, 0), (0, 0))
    assert disp._sink_blocks({"sol_h3_video_span": (0, 10)}, 10, "exact_kv", 64) == ((0, 0), (0, 0))


def _qkv(b=1, n=64, heads=2, d=128, dtype=torch.float32):
    g = torch.Generator().manual_seed(0)
    return [torch.randn(b, n, heads * d, generator=g).to(dtype) for _ in range(3)]


def dense_func(calls):
    from comfy.ldm.modules.attention import attention_pytorch

    def func(q, k, v, heads, **kw):
        calls.append("dense")
        return attention_pytorch(q, k, v, heads, **kw)
    return func


def test_override_gates(disp, monkeypatch):
    calls = []
    func = dense_func(calls)
    q, k, v = _qkv()
    ov = disp.make_override(tau=1.0, min_tokens=0, sigma_start=10.0, sigma_end=1.0,
                            dense_blocks=frozenset({3}))
    # mask -> dense
    ov(func, q, k, v, 2, mask=torch.zeros(64, 64))
    assert disp.sol_attn_stats()["dense_fallback"] == 1
    # dense block
    ov(func, q, k, v, 2, transformer_options={"sol_block": 3})
    assert disp.sol_attn_stats()["dense_block"] == 1
    # outside the sigma window (both sides)
    ov(func, q, k, v, 2, transformer_options={"sigmas": torch.tensor([20.0])})
    ov(func, q, k, v, 2, transformer_options={"sigmas": torch.tensor([0.5])})
    assert disp.sol_attn_stats()["outside_range"] == 2
    # inside the window: CPU tensors are ineligible ("not cuda") -> dense
    ov(func, q, k, v, 2, transformer_options={"sigmas": torch.tensor([5.0])})
    assert disp.sol_attn_stats()["dense_fallback"] == 2
    assert calls == ["dense"] * 5


def test_ineligible_reasons(disp, monkeypatch):
    monkeypatch.setattr(disp, "_sol_attn_kernel", object())
    q = torch.zeros(1, 64, 2, 128)
    assert disp._ineligible(q, q, None, 128, 0) == "not cuda"

    class FakeCuda:
        def __init__(self, t, dtype=torch.bfloat16):
            self.t, self.dtype, self.shape = t, dtype, t.shape
            self.device = torch.device("cuda", 0) if torch.cuda.is_available() else type("D", (), {"type": "cuda"})()
    assert "dtype" in disp._ineligible(FakeCuda(q, torch.float16), FakeCuda(q), None, 128, 0)
    assert "head_dim" in disp._ineligible(FakeCuda(q), FakeCuda(q), None, 64, 0)
    assert disp._ineligible(FakeCuda(q), FakeCuda(q), torch.ones(1), 128, 0) == "masked attention"
    assert "cross" in disp._ineligible(FakeCuda(q), FakeCuda(torch.zeros(1, 32, 2, 128)), None, 128, 0)
    assert "mismatch" in disp._ineligible(FakeCuda(q), FakeCuda(torch.zeros(1, 64, 1, 128)), None, 128, 0)
    assert "seq" in disp._ineligible(FakeCuda(q), FakeCuda(q), None, 128, 4096)
    assert disp._ineligible(FakeCuda(q), FakeCuda(q), None, 128, 0) is None
    monkeypatch.setattr(disp, "_sol_attn_kernel", None)
    assert disp._ineligible(q, q, None, 128, 0).startswith("kernel import failed")


def _force_sparse(disp, monkeypatch, kernel):
    monkeypatch.setattr(disp, "_ineligible", lambda *a: None)
    monkeypatch.setattr(disp, "_sol_attn_kernel", kernel)


def test_run_layouts_and_kernel_args(disp, monkeypatch):
    seen = {}

    def kernel(qs, ks, vs, **kw):
        seen.update(kw, shape=tuple(qs.shape), stride=qs.stride())
        return qs * 2
    _force_sparse(disp, monkeypatch, kernel)
    q, k, v = _qkv(n=64, heads=2)
    out = disp._run(q, k, v, 2, False, False, None, 0.7, 0, False, block=128,
                    sink_blocks=(0, 2), sink_q=(0, 1))
    assert seen["shape"] == (1, 64, 2, 128) and seen["tau"] == 0.7 and seen["block"] == 128
    assert seen["sink_blocks"] == (0, 2) and seen["sink_q"] == (0, 1)
    assert torch.equal(out, q * 2) and out.shape == q.shape
    # BHND in (skip_reshape) and out (skip_output_reshape): a transposed view, no copy
    qb = q.view(1, 64, 2, 128).transpose(1, 2)
    out = disp._run(qb, qb, qb, 2, True, True, None, 1.0, 0, False)
    assert seen["shape"] == (1, 64, 2, 128) and seen["stride"] == q.view(1, 64, 2, 128).stride()
    assert torch.equal(out, qb * 2)
    assert disp.sol_attn_stats()["sparse"] == 2


def test_int8_dispatch(disp, monkeypatch):
    seen = {}
    _force_sparse(disp, monkeypatch, lambda *a, **kw: None)
    monkeypatch.setattr(disp, "_sol_attn_int8_kernel",
                        lambda qs, ks, vs, **kw: seen.update(kw) or qs)
    q, k, v = _qkv()
    disp._run(q, k, v, 2, False, False, 0.1, 1.0, 0, False, int8_qk=True, int8_pv=False)
    assert seen["int8_pv"] is False and seen["scale"] == 0.1 and seen["pv_codes"] == "block"
    # the running-max P codes reach the kernel from the override's policy
    seen.clear()
    ov = disp.make_override(min_tokens=0, int8_qk=True, pv_codes="running")
    assert ov.policy.pv_codes == "running"
    disp._run(q, k, v, 2, False, False, 0.1, 1.0, 0, False, int8_qk=True, pv_codes="running")
    assert seen["pv_codes"] == "running"


def test_kernel_error_falls_back_dense(disp, monkeypatch):
    def boom(*a, **kw):
        raise RuntimeError("kernel exploded")
    _force_sparse(disp, monkeypatch, boom)
    calls = []
    q, k, v = _qkv()
    out = disp.make_override(min_tokens=0)(dense_func(calls), q, k, v, 2)
    assert calls == ["dense"] and out.shape == q.shape
    assert disp.sol_attn_stats()["errors"] == 1


def test_previous_override_is_chained(disp):
    calls = []

    def previous(func, q, k, v, heads, **kw):
        calls.append("previous")
        return func(q, k, v, heads, **kw)
    q, k, v = _qkv()
    disp.make_override(min_tokens=0, previous=previous)(dense_func(calls), q, k, v, 2,
                                                       mask=torch.zeros(64, 64))
    assert calls == ["previous", "dense"]


def test_tau_profile_per_block(disp, monkeypatch):
    seen = []
    _force_sparse(disp, monkeypatch, lambda qs, ks, vs, **kw: seen.append(kw["tau"]) or qs)
    q, k, v = _qkv()
    ov = disp.make_override(tau=1.3, min_tokens=0, tau_profile={2: 0.5})
    ov(None, q, k, v, 2, transformer_options={"sol_block": 2})
    ov(None, q, k, v, 2, transformer_options={"sol_block": 5})
    assert seen == [0.5, 1.3]


def test_probe_records_and_returns_dense(disp):
    calls = []
    q, k, v = _qkv()
    inner = disp.make_override(min_tokens=0)
    probe = disp.make_probe_override(inner)
    disp._probe.clear()
    out = probe(dense_func(calls), q, k, v, 2, transformer_options={"sol_block": 4})
    assert calls == ["dense", "dense"]  # inner fell back (CPU), then the reference
    assert 4 in disp._probe and disp._probe[4][1] == 1
    disp.log_probe_summary()
    assert not disp._probe
    assert out.shape == q.shape


def test_block_index_publisher(disp):
    class Block(torch.nn.Module):
        def forward(self, x, transformer_options=None):
            self.seen = dict(transformer_options)
            return x

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([Block(), Block()])
    m = Model()
    assert disp._install_block_index(m)
    opts = {}
    for blk in m.blocks:
        blk(torch.zeros(1), transformer_options=opts)
    assert [blk.seen["sol_block"] for blk in m.blocks] == [0, 1]
    assert not disp._install_block_index(torch.nn.Linear(1, 1))


class _Sampling:
    def percent_to_sigma(self, p):
        return 10.0 * (1.0 - p)


class _Patcher:
    def __init__(self, diffusion_model):
        self.dm = diffusion_model
        self.model_options = {"transformer_options": {}}
        self.object_patches = {}
        self.callbacks = []

    def get_model_object(self, name):
        return {"diffusion_model": self.dm, "model_sampling": _Sampling()}[name]

    def clone(self):
        c = _Patcher(self.dm)
        c.model_options = {"transformer_options": dict(self.model_options["transformer_options"])}
        c.object_patches = dict(self.object_patches)
        return c

    def add_object_patch(self, key, obj):
        self.object_patches[key] = obj

    def add_callback(self, kind, fn):
        self.callbacks.append((kind, fn))


def test_patch_node_execute(pkg, monkeypatch):
    d = importlib.import_module(f"{pkg.__name__}._dispatch")
    if pkg._sol_attn_kernel is None:
        pytest.skip(f"libsolattn.so not importable here: {pkg._IMPORT_ERROR}")

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([torch.nn.Identity() for _ in range(4)])
    m = _Patcher(Model())
    (out,) = pkg.SolAttnPatch.execute(m, tau=1.1, start_percent=0.2, end_percent=0.9,
                                      min_tokens=1024, int8_qk=False, sink_conditioning="off",
                                      morton=True, morton_curve="3d", dense_blocks="0,-1",
                                      verbose=False, tau_profile="1=0.5", block_size="128")
    opts = out.model_options["transformer_options"]
    assert callable(opts["optimized_attention_override"])
    assert opts["sol_compose"] == {"sigma_start": 8.0, "sigma_end": pytest.approx(1.0),
                                   "min_tokens": 1024}
    assert opts["sol_block_size"] == 128
    assert "sol_morton" not in opts  # neither Wan nor H3: Morton skipped
    assert m.model_options["transformer_options"] == {}  # the input model is untouched
    # the probe wraps it
    (probed,) = pkg.SolAttnBlockProbe.execute(out)
    assert probed.callbacks and probed.callbacks[0][0] == "on_cleanup"
    assert d.sol_attn_stats()["sparse"] == 0
