"""Composition with object-patched attention forwards, the SOL_ATTN global
override and the block-count eligibility gate, on the CPU. A tensor subclass
that reports a GPU device stands in for a bf16 GPU activation (nothing here
computes on it)."""

import importlib

import pytest
import torch


class GpuLike(torch.Tensor):
    """Reports device cuda:0; used only for the gates' type/shape checks."""

    @property
    def device(self):
        return torch.device("cuda", 0)


def gpu_like(*shape, dtype=torch.bfloat16):
    return torch.zeros(*shape, dtype=dtype).as_subclass(GpuLike)


@pytest.fixture
def comp(pkg):
    return importlib.import_module(f"{pkg.__name__}._compose")


class Attn(torch.nn.Module):
    calls = []

    def forward(self, x, transformer_options=None):
        Attn.calls.append("stock")
        return "stock"


def _patched(x, transformer_options=None):
    Attn.calls.append("patched")
    return "patched"


GATE = {"sigma_start": 8.0, "sigma_end": 1.0, "min_tokens": 1024}


@pytest.fixture(autouse=True)
def _clear():
    Attn.calls.clear()


def test_gate_routes_eligible_calls_to_stock_forward(comp):
    fwd = comp._compose_module_patch(Attn(), _patched)
    assert fwd._sol_composed
    opts = {"sol_compose": GATE, "sigmas": torch.tensor([5.0])}
    assert fwd(gpu_like(1, 2048, 64), transformer_options=opts) == "stock"
    # H3 layout: tokens first
    assert fwd(gpu_like(2048, 64), transformer_options=opts) == "stock"
    refused = [
        (gpu_like(1, 512, 64), opts),                                   # too short
        (gpu_like(1, 2048, 64), {**opts, "sigmas": torch.tensor([9.0])}),  # before the window
        (gpu_like(1, 2048, 64), {**opts, "sigmas": torch.tensor([0.5])}),  # after it
        (gpu_like(1, 2048, 64, dtype=torch.float16), opts),              # not bf16
        (torch.zeros(1, 2048, 64, dtype=torch.bfloat16), opts),          # not on the GPU
        (gpu_like(1, 1, 2048, 64), opts),                                # 4-D
        (gpu_like(1, 2048, 64), {"sigmas": torch.tensor([5.0])}),        # no gate published
    ]
    for x, o in refused:
        assert fwd(x, transformer_options=o) == "patched"
    # gate found among positional dicts when transformer_options is not a kwarg
    assert fwd(gpu_like(1, 2048, 64), {"sol_compose": GATE}) == "stock"
    assert Attn.calls == ["stock", "stock"] + ["patched"] * len(refused) + ["stock"]


def test_handoff_list_is_consumed_and_delegate_preferred(comp):
    module = Attn()
    fwd = comp._compose_module_patch(module, _patched)
    x = gpu_like(1, 2048, 64)
    box = [x]
    seen = {}

    def stock(self, t, transformer_options=None):
        seen["arg"] = t
        return "stock"
    module_type_forward = Attn.forward
    try:
        Attn.forward = stock
        fwd = comp._compose_module_patch(module, _patched)
        assert fwd(box, transformer_options={"sol_compose": GATE}) == "stock"
    finally:
        Attn.forward = module_type_forward
    assert box == [] and seen["arg"] is x
    delegated = []
    opts = {"sol_compose": GATE, "sol_take_forward": lambda m, *a, **k: delegated.append(m) or "own"}
    assert fwd(gpu_like(1, 2048, 64), transformer_options=opts) == "own"
    assert delegated == [module]


def test_compose_hooks_wrap_foreign_forwards_at_run_time(comp):
    class Block(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.self_attn = Attn()

        def forward(self, x):
            return self.self_attn.forward(x, transformer_options={"sol_compose": GATE})

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([Block(), Block(), Block()])

    model = Model()
    comp._install_compose_hooks(model, "self_attn")
    comp._install_compose_hooks(model, "self_attn")  # once per model
    a0, a1, a2 = (b.self_attn for b in model.blocks)
    a0.forward = _patched                               # a foreign patch, applied later
    a1.forward = a1.forward                             # stock forward bound on the instance

    def routed(x, transformer_options=None):
        return "routed"
    routed._uses_optimized_attention = True
    a2.forward = routed                                 # reaches optimized_attention itself
    for blk in model.blocks:
        blk(gpu_like(1, 2048, 64))
    assert isinstance(a0.__dict__["forward"], comp.ComposedForward)
    assert not isinstance(a1.__dict__["forward"], comp.ComposedForward)
    assert a2.__dict__["forward"] is routed
    # the wrapped one now gives eligible calls to the stock forward
    assert Attn.calls == ["stock", "stock"]


def test_node_composes_self_attention_object_patches(pkg):
    from test_nodes import _Patcher

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([torch.nn.Identity()])

        def rope_encode(self):
            pass

    if pkg._sol_attn_kernel is None:
        pytest.skip(f"libsolattn.so not importable here: {pkg._IMPORT_ERROR}")
    patcher = _Patcher(Model())
    modules = {}

    def get(name):
        if name in ("diffusion_model", "model_sampling"):
            return _Patcher.get_model_object(patcher, name)
        return modules.setdefault(name, Attn())
    patcher.get_model_object = get
    keep = lambda *a, **k: "keep"  # noqa: E731
    routed = lambda *a, **k: "routed"  # noqa: E731
    routed._uses_optimized_attention = True
    patcher.object_patches = {
        "diffusion_model.blocks.0.self_attn.forward": keep,
        "diffusion_model.blocks.0.cross_attn.forward": keep,
        "diffusion_model.blocks.0.attn2.forward": keep,
        "diffusion_model.blocks.1.self_attn.forward": routed,
        "diffusion_model.blocks.0.norm.weight": keep,
    }
    orig_clone = patcher.clone

    def clone():
        c = orig_clone()
        c.get_model_object = get
        return c
    patcher.clone = clone
    (out,) = pkg.SolAttnPatch.execute(patcher, tau=1.0, start_percent=0.2, end_percent=0.9,
                                      min_tokens=1024, int8_qk=False, sink_conditioning="off",
                                      morton=False, morton_curve="3d", dense_blocks="",
                                      verbose=False)
    comp = importlib.import_module(f"{pkg.__name__}._compose")
    patches = out.object_patches
    assert isinstance(patches["diffusion_model.blocks.0.self_attn.forward"], comp.ComposedForward)
    for key in ("diffusion_model.blocks.0.cross_attn.forward", "diffusion_model.blocks.0.attn2.forward",
                "diffusion_model.blocks.0.norm.weight"):
        assert patches[key] is keep
    assert patches["diffusion_model.blocks.1.self_attn.forward"] is routed
    assert patcher.object_patches["diffusion_model.blocks.0.self_attn.forward"] is keep


def test_sol_attn_env_installs_global_override(pkg, monkeypatch):
    import comfy.ldm.modules.attention as attention

    monkeypatch.setattr(attention, "optimized_attention", attention.optimized_attention)
    monkeypatch.setattr(attention, "optimized_attention_masked", attention.optimized_attention_masked)
    for off in ({}, {"SOL_ATTN": "0"}, {"SOL_ATTN": ""}, {"SOL_ATTN": "false"}):
        assert pkg._install_global_override(off) is False
    assert attention.optimized_attention is not pkg.attention_sol
    if pkg._sol_attn_kernel is not None:
        assert pkg._install_global_override({"SOL_ATTN": "1"}) is True
        assert attention.optimized_attention is pkg.attention_sol
        assert attention.optimized_attention_masked is pkg.attention_sol
    monkeypatch.setattr(pkg, "_sol_attn_kernel", None)
    monkeypatch.setattr(attention, "optimized_attention", None)
    assert pkg._install_global_override({"SOL_ATTN": "1"}) is False
    assert attention.optimized_attention is None


def test_attention_sol_falls_back_on_cpu(pkg):
    g = torch.Generator().manual_seed(0)
    q, k, v = (torch.randn(1, 64, 2 * 128, generator=g) for _ in range(3))
    d = importlib.import_module(f"{pkg.__name__}._dispatch")
    d.reset_sol_attn_stats()
    out = pkg.attention_sol(q, k, v, 2)
    from comfy.ldm.modules.attention import attention_pytorch
    assert torch.allclose(out, attention_pytorch(q, k, v, 2))
    assert d.sol_attn_stats()["dense_fallback"] == 1  # CPU tensors: "not cuda"
    out = pkg.attention_sol(q, k, v, 2, mask=torch.zeros(64, 64))
    assert d.sol_attn_stats()["dense_fallback"] == 1  # masked: never tried


def test_long_sequences_are_ineligible_not_errors(pkg, monkeypatch):
    d = importlib.import_module(f"{pkg.__name__}._dispatch")
    monkeypatch.setattr(d, "_sol_attn_kernel", object())
    d.reset_sol_attn_stats()
    for block in (64, 128):
        limit = d.MAX_BLOCKS * block
        ok = gpu_like(1, limit, 2, 128)
        assert d._ineligible(ok, ok, None, 128, 0, block) is None
        long = gpu_like(1, limit + 1, 2, 128)
        reason = d._ineligible(long, long, None, 128, 0, block)
        assert reason is not None and "blocks" in reason
    # through the override: counted as a dense fallback, not an error
    calls = []
    q = gpu_like(1, d.MAX_BLOCKS * 64 + 1, 2 * 128)
    ov = d.make_override(min_tokens=0, block=64)
    ov(lambda *a, **kw: calls.append("dense"), q, q, q, 2)
    assert calls == ["dense"]
    assert d.sol_attn_stats()["dense_fallback"] == 1 and d.sol_attn_stats()["errors"] == 0
