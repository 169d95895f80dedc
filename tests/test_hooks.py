"""Model-level Morton hooks on the CPU, with small stand-in Wan and MiniMax-H3
models. The row gather is swapped for ``index_select`` (the product's gather
kernel needs a GPU; ``tests/test_gpu_parity.py`` runs the same hooks through
it). Checked: a single decision point per pass, tokens and RoPE table permuted
together, order restored after the last block, neutrality for dense
attention, the H3 span roll onto the block grid and the publication of
``sol_h3_video_span``."""

import importlib
import sys
import types

import pytest
import torch


def _index_gather(x, index, dim):
    return x.index_select(dim, index.to(x.device))


@pytest.fixture
def wan(pkg, monkeypatch):
    mod = importlib.import_module(f"{pkg.__name__}._morton")
    monkeypatch.setattr(mod, "_gather", _index_gather)
    return mod


@pytest.fixture
def h3(pkg, monkeypatch):
    mod = importlib.import_module(f"{pkg.__name__}._morton_h3")
    monkeypatch.setattr(mod, "_gather", _index_gather)
    return mod


def _attend(x, table):
    """Dense attention whose keys carry a per-token table row: equivariant
    under a permutation applied to tokens and table rows together."""
    xd = x.double()
    qk = xd * table.double()
    w = torch.softmax(qk @ qk.transpose(-1, -2) / x.shape[-1] ** 0.5, dim=-1)
    return (xd + w @ xd).to(x.dtype)


# ----------------------------------------------------------------- Wan
class WanBlock(torch.nn.Module):
    def __init__(self, log):
        super().__init__()
        self.log = log

    def forward(self, x, freqs=None, transformer_options=None):
        self.log.append(freqs)
        return _attend(x, freqs[0])


class WanModel(torch.nn.Module):
    def __init__(self, n=3):
        super().__init__()
        self.seen = []
        self.blocks = torch.nn.ModuleList([WanBlock(self.seen) for _ in range(n)])

    def rope_encode(self):  # marks the model Wan-style for the node
        pass

    def forward(self, x, freqs, options):
        self.seen.clear()
        for blk in self.blocks:
            x = blk(x, freqs=freqs, transformer_options=options)
        return x


def _wan_inputs(grid, c=16, seed=0):
    g = torch.Generator().manual_seed(seed)
    n = grid[0] * grid[1] * grid[2]
    return torch.randn(2, n, c, generator=g), torch.rand(1, n, c, generator=g) + 0.5


def test_wan_reorder_is_neutral_and_permutes_table(wan):
    grid = (3, 4, 6)
    model = WanModel()
    wan.install_wan_morton(model)
    wan.install_wan_morton(model)  # idempotent: one set of hooks
    x, freqs = _wan_inputs(grid)
    plain = model(x, freqs, {"grid_sizes": grid})
    assert all(f is freqs for f in model.seen)
    opts = {"grid_sizes": grid, "sol_morton": True, "sol_morton_curve": "3d"}
    hooked = model(x, freqs, opts)
    perm, inverse = wan.morton_perm(grid, "cpu", "3d")
    assert not torch.equal(perm, torch.arange(perm.numel()))
    # every block saw the permuted table, built once
    assert all(torch.equal(f, freqs[:, perm]) for f in model.seen)
    assert all(f is model.seen[0] for f in model.seen)
    torch.testing.assert_close(hooked, plain, rtol=1e-6, atol=1e-6)


def test_wan_block_stack_runs_in_morton_order(wan):
    """Inside the stack the tokens are in Morton order; outside, in raster order."""
    grid = (2, 4, 4)
    seen_x = []

    class Probe(WanBlock):
        def forward(self, x, freqs=None, transformer_options=None):
            seen_x.append(x.clone())
            return x + 1.0

    model = WanModel(2)
    model.blocks[0] = Probe(model.seen)
    wan.install_wan_morton(model)
    x, freqs = _wan_inputs(grid)
    out = model(x, freqs, {"grid_sizes": grid, "sol_morton": True, "sol_morton_curve": "2d_frame"})
    perm, _ = wan.morton_perm(grid, "cpu", "2d_frame")
    assert torch.equal(seen_x[0], x[:, perm])
    # restored: block 1 added the table-weighted attention in Morton order, undone after
    ref = WanModel(2)
    ref.blocks[0] = Probe(ref.seen)
    torch.testing.assert_close(out, ref(x, freqs, {"grid_sizes": grid}), rtol=1e-6, atol=1e-6)


@pytest.mark.parametrize("case", ["flag_off", "no_grid", "extra_tokens", "table_mismatch"])
def test_wan_inactive_cases_leave_pass_untouched(wan, case):
    grid = (2, 4, 4)
    model = WanModel(2)
    wan.install_wan_morton(model)
    x, freqs = _wan_inputs(grid)
    opts = {"grid_sizes": grid, "sol_morton": True}
    if case == "flag_off":
        opts["sol_morton"] = False
    elif case == "no_grid":
        del opts["grid_sizes"]
    elif case == "extra_tokens":  # a reference latent prepended: tokens != grid
        x = torch.cat([x[:, :5], x], dim=1)
        freqs = torch.cat([freqs[:, :5], freqs], dim=1)
    else:
        freqs = freqs[:, :-1]
        x = x[:, :-1]
        opts["grid_sizes"] = grid  # x no longer matches either
    out = model(x, freqs, opts)
    assert all(f is freqs for f in model.seen)
    torch.testing.assert_close(out, WanModel(2)(x, freqs, {}), rtol=0, atol=0)


def test_wan_state_does_not_leak_between_passes(wan):
    grid = (2, 4, 4)
    model = WanModel(2)
    wan.install_wan_morton(model)
    x, freqs = _wan_inputs(grid)
    model(x, freqs, {"grid_sizes": grid, "sol_morton": True})
    # next pass with the flag off: no stale table, no stale inverse
    out = model(x, freqs, {"grid_sizes": grid})
    assert all(f is freqs for f in model.seen)
    torch.testing.assert_close(out, WanModel(2)(x, freqs, {}), rtol=0, atol=0)


# ------------------------------------------------------------------ H3
def _h3_module():
    """A stand-in for the H3 model module: PackedLayout + the diffusion model."""
    mod = types.ModuleType("fake_h3_model")

    class PackedLayout:
        def __init__(self, text_len, latent_t, latent_h, latent_w, audio_t, ref_len=0,
                     video_rows=None):
            video = latent_t * (latent_h // 2) * (latent_w // 2) if video_rows is None else video_rows
            cond = text_len + ref_len + audio_t
            self.segments = [(0, text_len, "text"), (text_len, cond, "audio"),
                             (cond, cond + video, "video")]
            self.position_ids = torch.arange(cond + video)

    class Block(torch.nn.Module):
        def __init__(self, log):
            super().__init__()
            self.log = log

        def forward(self, h, t_emb, mod_segments, rope, extra=None):
            self.log.append(rope)
            return _attend(h, rope[0])

    class H3(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.seen = []
            self.published = []
            self.blocks = torch.nn.ModuleList([Block(self.seen) for _ in range(3)])

        def rope_freqs(self, position_ids, device):
            g = torch.Generator().manual_seed(int(position_ids.numel()))
            return torch.rand(1, position_ids.numel(), 8, generator=g) + 0.5

        def _forward(self, x, timestep, context, transformer_options={}, layout_args=None):
            self.seen.clear()
            layout = sys.modules[type(self).__module__].PackedLayout(*layout_args)
            rope = self.rope_freqs(layout.position_ids, x.device)
            self.published.append(transformer_options.get("sol_h3_video_span"))
            h = x
            for blk in self.blocks:
                h = blk(h, None, None, rope)
            return h

    mod.PackedLayout, mod.H3 = PackedLayout, H3
    H3.__module__ = mod.__name__
    sys.modules[mod.__name__] = mod
    return mod


@pytest.mark.parametrize("block", [64, 128])
@pytest.mark.parametrize("text_len", [64, 37])  # aligned and ragged span starts
def test_h3_reorder_neutral_roll_and_span(h3, block, text_len):
    mod = _h3_module()
    model = mod.H3()
    h3.install_h3_morton(model, block=64)
    layout_args = (text_len, 4, 16, 16, 10)  # video 4x8x8 = 256 rows after 10 audio rows
    S = text_len + 10 + 256
    g = torch.Generator().manual_seed(1)
    x = torch.randn(S, 8, generator=g)
    opts = {}
    plain = model._forward(x, None, None, transformer_options=opts, layout_args=layout_args)
    start, stop = text_len + 10, S
    assert model.published == [(start, stop)]      # published during the pass
    assert "sol_h3_video_span" not in opts          # and removed after it
    assert all(r is model.seen[0] for r in model.seen)
    table = model.seen[0]

    opts = {"sol_morton": True, "sol_morton_curve": "3d", "sol_block_size": block}
    hooked = model._forward(x, None, None, transformer_options=opts, layout_args=layout_args)
    fwd, inv = h3._composed((4, 8, 8), "3d", x.device, start, stop, S, block)
    perm, _ = h3.morton_perm((4, 8, 8), "cpu", "3d")
    pad = (-start) % block
    # identity outside the span, the rotated Morton order inside
    assert torch.equal(fwd[:start], torch.arange(start))
    assert torch.equal(fwd[start:], torch.roll(perm, pad) + start)
    assert torch.equal(fwd[inv], torch.arange(S))
    assert all(torch.equal(r, table[:, fwd]) for r in model.seen)
    torch.testing.assert_close(hooked, plain, rtol=1e-6, atol=1e-6)
    if pad:
        # the first full block after the span start holds a whole Z-order cell group:
        # rotated rows begin at the next block boundary
        assert torch.equal(fwd[start + pad:start + pad + 8], perm[:8] + start)


def test_h3_sink_publication_without_morton_and_unregistered_ids(h3):
    mod = _h3_module()
    model = mod.H3()
    h3.install_h3_morton(model)
    x = torch.randn(64 + 10 + 72, 8)
    out = model._forward(x, None, None, transformer_options={}, layout_args=(64, 3, 8, 12, 10))
    assert model.published == [(74, 146)]
    assert all(r is model.seen[0] for r in model.seen)  # not reordered
    # a position_ids tensor no layout registered: nothing published
    model.published.clear()
    table = model.rope_freqs(torch.arange(146), "cpu")
    assert table.shape == (1, 146, 8)
    assert out.shape == x.shape


def test_h3_grid_mismatch_keeps_order(h3):
    """A video segment that is not the patchified latent grid publishes its
    bounds (the sink still applies) but is never reordered."""
    mod = _h3_module()
    model = mod.H3()
    h3.install_h3_morton(model)
    layout = mod.PackedLayout(64, 3, 8, 12, 10, video_rows=70)
    bounds, span = h3._SPANS.lookup(layout.position_ids)
    assert bounds == (74, 144) and span is None
    assert h3._SPANS.lookup(torch.arange(144)) is None  # same values, other tensor

    class Layout70(mod.PackedLayout):
        def __init__(self, *args):
            super().__init__(*args, video_rows=70)

    x = torch.randn(144, 8)
    opts = {"sol_morton": True}
    mod.PackedLayout = Layout70  # the model builds layouts through its module
    out = model._forward(x, None, None, transformer_options=opts, layout_args=(64, 3, 8, 12, 10))
    assert model.published == [(74, 144)]
    assert all(r is model.seen[0] for r in model.seen)  # not reordered
    torch.testing.assert_close(out, mod.H3()._forward(x, None, None, layout_args=(64, 3, 8, 12, 10)),
                               rtol=0, atol=0)


def test_hooks_on_host_tensors_use_index_select(pkg):
    """With Morton on and the pass's tensors on the host, the hooks' own gather
    (not the kernel, which needs device tensors) permutes them: the Wan and H3
    stand-ins give the un-hooked outputs, and the blocks saw permuted tables."""
    wan = importlib.import_module(f"{pkg.__name__}._morton")
    h3 = importlib.import_module(f"{pkg.__name__}._morton_h3")
    grid = (2, 4, 6)
    model = WanModel(2)
    wan.install_wan_morton(model)
    x, freqs = _wan_inputs(grid, seed=3)
    plain = WanModel(2)(x, freqs, {})
    hooked = model(x, freqs, {"grid_sizes": grid, "sol_morton": True, "sol_morton_curve": "3d"})
    perm, _ = wan.morton_perm(grid, "cpu", "3d")
    assert all(torch.equal(f, freqs[:, perm]) for f in model.seen)
    torch.testing.assert_close(hooked, plain, rtol=1e-6, atol=1e-6)

    mod = _h3_module()
    m3 = mod.H3()
    h3.install_h3_morton(m3)
    layout_args = (37, 4, 16, 16, 10)
    x3 = torch.randn(37 + 10 + 256, 8, generator=torch.Generator().manual_seed(4))
    ref3 = mod.H3()._forward(x3, None, None, layout_args=layout_args)
    out3 = m3._forward(x3, None, None, transformer_options={"sol_morton": True, "sol_block_size": 64},
                       layout_args=layout_args)
    table = mod.H3().rope_freqs(torch.arange(x3.shape[0]), "cpu")
    assert m3.seen and not torch.equal(m3.seen[0], table)  # the blocks saw the permuted table
    torch.testing.assert_close(out3, ref3, rtol=1e-6, atol=1e-6)
