"""The drop-in path on the device: ComfyUI's override protocol with real GPU
tensors through SolAttnOverride -> _run -> the HIP kernels -> restore, in both
layouts ComfyUI passes ([B, N, heads*dim] and a genuinely contiguous
[B, H, N, D] with skip_reshape / skip_output_reshape), the Patch Sol-Attn
node's override, the "sol_attn" registry entry, the MiniMax-H3 conditioning
sink and the H3 Morton hooks through the gather kernel.

Each sparse answer must be bit-identical to the kernel-level call on the BTHD
tensors (the layout adaptation copies nothing and changes no arithmetic) and
agree per query block with the oracle's restatement of the reference loop
(BF16: max-abs 2e-2, cosine >= 0.9995; INT8: cosine >= 0.999).
Reference: /root/reference/__init__.py:192-231 (_run), 256-320 (override),
649-663 (attention_sol), /root/reference/_morton_h3.py:161-218 (H3 hooks).
"""

import importlib
import sys
import types

import numpy as np
import pytest
import torch

import oracle
from _util import bits, check_int8_blocks, compare_rows, cosine, per_block
from test_nodes import _Patcher

pytestmark = pytest.mark.gpu

BF16_MAXABS, BF16_COS = 2e-2, 0.9995
MODES = {
    "bf16": dict(int8_qk=False),
    "int8_pv": dict(int8_qk=True, int8_pv=True),
    "int8_pv_running": dict(int8_qk=True, int8_pv=True, pv_codes="running"),
    "int8_bf16pv": dict(int8_qk=True, int8_pv=False),
}


def _mods(pkg):
    n = pkg.__name__
    return (importlib.import_module(f"{n}._dispatch"), importlib.import_module(f"{n}._tri_fwd"),
            importlib.import_module(f"{n}._int8_fwd"))


def _field(N, H, seed):
    """[1, N, H, 128] bf16 on the host: a field constant over runs of 48 tokens
    plus noise, so routing keeps some blocks and pools others."""
    g = torch.Generator().manual_seed(seed)
    base = torch.randn(1, N // 48 + 1, H, 128, generator=g).repeat_interleave(48, dim=1)[:, :N]
    return (base + 0.6 * torch.randn(1, N, H, 128, generator=g)).to(torch.bfloat16)


def _direct(pkg, q, k, v, mode, **kw):
    """The kernel-level call on BTHD tensors."""
    _, tri, i8 = _mods(pkg)
    if mode == "bf16":
        return tri.sol_attn(q, k, v, **kw)
    return i8.sol_attn_int8(q, k, v, int8_pv=MODES[mode]["int8_pv"],
                            pv_codes=MODES[mode].get("pv_codes", "block"), **kw)


def _against_oracle(label, got, hq, hk, hv, mode, block, tau, sink_kv=(0, 0), sink_q=(0, 0)):
    """Every query block of `got` [1, N, H, 128] against the oracle loops."""
    qb, kb, vb = bits(hq), bits(hk), bits(hv)
    int8 = mode != "bf16"
    pv = MODES[mode].get("int8_pv", True)
    ref = oracle.prepare(qb, kb, vb, block=block, tau=tau, int8=int8, int8_pv=pv,
                         sink_kv=sink_kv, sink_q=sink_q)
    H = qb.shape[2]
    rows = [(0, h, i) for h in range(H) for i in range(ref["NT"])]
    out = got.float().cpu().numpy()
    if int8:
        check_int8_blocks(label, out, qb, vb, ref, rows, pv, block,
                          pv_codes=MODES[mode].get("pv_codes", "block"))
        return
    port = oracle.forward_port(qb, kb, vb, ref, rows)
    err, cos = compare_rows(out, port, block)
    worst = min(s[2] for s in per_block(out, port, block))
    print(f"[{label}] {len(rows)} query blocks: max|err|={err:.3e} cos={cos:.6f} worst block "
          f"cos {worst:.6f}", flush=True)
    assert err < BF16_MAXABS and cos >= BF16_COS and worst >= BF16_COS


def _dense(calls):
    from comfy.ldm.modules.attention import attention_pytorch

    def func(q, k, v, heads, **kw):
        calls.append("dense")
        return attention_pytorch(q, k, v, heads, **kw)
    return func


@pytest.mark.parametrize("block", [64, 128])
@pytest.mark.parametrize("mode", list(MODES))
def test_override_in_both_comfy_layouts(pkg, dev, mode, block):
    """make_override(...) on device tensors: [B, N, H*D] in and out, then a
    contiguous BHND tensor (token stride 128, head stride N*128) with
    skip_reshape and skip_output_reshape, then BHND in and [B, N, H*D] out."""
    disp = _mods(pkg)[0]
    N, H, tau = 1100, 3, 0.9
    print(f"[override] mode={mode} block={block} N={N} H={H}", flush=True)
    hq, hk, hv = _field(N, H, 1), _field(N, H, 2), _field(N, H, 3)
    q, k, v = (t.to(dev) for t in (hq, hk, hv))
    direct = _direct(pkg, q, k, v, mode, tau=tau, block=block)
    disp.reset_sol_attn_stats()
    ov = disp.make_override(tau=tau, min_tokens=0, block=block, **MODES[mode])
    calls = []

    flat = [t.reshape(1, N, H * 128) for t in (q, k, v)]
    out = ov(_dense(calls), *flat, H)
    assert out.shape == (1, N, H * 128)
    assert torch.equal(out.view(1, N, H, 128), direct)

    bhnd = [t.transpose(1, 2).contiguous() for t in (q, k, v)]
    assert bhnd[0].stride() == (H * N * 128, N * 128, 128, 1)
    out = ov(_dense(calls), *bhnd, H, skip_reshape=True, skip_output_reshape=True)
    assert out.shape == (1, H, N, 128)
    assert torch.equal(out.transpose(1, 2), direct)

    out = ov(_dense(calls), *bhnd, H, skip_reshape=True, skip_output_reshape=False)
    assert out.shape == (1, N, H * 128)
    assert torch.equal(out.view(1, N, H, 128), direct)

    torch.cuda.synchronize()
    assert calls == [] and disp.sol_attn_stats()["sparse"] == 3
    assert disp.sol_attn_stats()["errors"] == 0
    _against_oracle(f"override {mode} block {block}", direct, hq, hk, hv, mode, block, tau)


@pytest.mark.parametrize("int8_qk", [False, True])
def test_patch_node_override_on_device(pkg, dev, int8_qk):
    """The override the Patch Sol-Attn node installs: inside the sigma window
    the call is sparse and equals the kernel-level call bit for bit; outside
    it, and for a dense block, ComfyUI's attention answers."""
    disp = _mods(pkg)[0]

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.blocks = torch.nn.ModuleList([torch.nn.Identity() for _ in range(3)])
    (patched,) = pkg.SolAttnPatch.execute(
        _Patcher(Model()), tau=1.1, start_percent=0.2, end_percent=0.9, min_tokens=1024,
        int8_qk=int8_qk, sink_conditioning="off", morton=False, morton_curve="3d",
        dense_blocks="2", verbose=False, int8_pv=True, block_size="128")
    ov = patched.model_options["transformer_options"]["optimized_attention_override"]
    N, H = 1500, 2
    print(f"[node] int8_qk={int8_qk} N={N} H={H}", flush=True)
    hq, hk, hv = _field(N, H, 11), _field(N, H, 12), _field(N, H, 13)
    q, k, v = (t.to(dev) for t in (hq, hk, hv))
    mode = "int8_pv" if int8_qk else "bf16"
    direct = _direct(pkg, q, k, v, mode, tau=1.1, block=128)
    flat = [t.reshape(1, N, H * 128) for t in (q, k, v)]
    calls = []
    inside = {"sigmas": torch.tensor([5.0]), "sol_block": 0}
    out = ov(_dense(calls), *flat, H, transformer_options=inside)
    assert calls == [] and torch.equal(out.view(1, N, H, 128), direct)
    ref = _dense([])(*flat, H).float()
    for opts in ({"sigmas": torch.tensor([9.5]), "sol_block": 0},   # before the window
                 {"sigmas": torch.tensor([5.0]), "sol_block": 2}):  # a dense block
        out = ov(_dense(calls), *flat, H, transformer_options=opts)
        assert (out.float() - ref).abs().max().item() <= 1e-2  # ComfyUI's dense SDPA
    torch.cuda.synchronize()
    stats = disp.sol_attn_stats()
    assert calls == ["dense", "dense"]
    assert stats["sparse"] == 1 and stats["outside_range"] == 1 and stats["dense_block"] == 1
    _against_oracle(f"node int8_qk={int8_qk}", direct, hq, hk, hv, mode, 128, 1.1)


def test_attention_sol_registry_entry(pkg, dev):
    """"sol_attn" in ComfyUI's registry: from 4096 tokens the sparse path with
    the registry defaults (tau 1.0, block 64, BF16) in both layouts; shorter
    calls and masked calls are ComfyUI's dense attention."""
    disp = _mods(pkg)[0]
    from comfy.ldm.modules.attention import attention_pytorch
    N, H = 4160, 2
    print(f"[attention_sol] N={N} H={H}", flush=True)
    hq, hk, hv = _field(N, H, 21), _field(N, H, 22), _field(N, H, 23)
    q, k, v = (t.to(dev) for t in (hq, hk, hv))
    direct = _direct(pkg, q, k, v, "bf16", tau=1.0, block=64)
    disp.reset_sol_attn_stats()
    flat = [t.reshape(1, N, H * 128) for t in (q, k, v)]
    assert torch.equal(pkg.attention_sol(*flat, H).view(1, N, H, 128), direct)
    bhnd = [t.transpose(1, 2).contiguous() for t in (q, k, v)]
    out = pkg.attention_sol(*bhnd, H, skip_reshape=True, skip_output_reshape=True)
    assert torch.equal(out.transpose(1, 2), direct)
    short = [t[:, :4000] for t in flat]
    assert torch.equal(pkg.attention_sol(*short, H), attention_pytorch(*short, H))
    mask = torch.zeros(N, N, device=dev)
    assert torch.equal(pkg.attention_sol(*flat, H, mask=mask), attention_pytorch(*flat, H, mask=mask))
    torch.cuda.synchronize()
    stats = disp.sol_attn_stats()
    assert stats["sparse"] == 2 and stats["dense_fallback"] == 1 and stats["errors"] == 0
    _against_oracle("attention_sol", direct, hq, hk, hv, "bf16", 64, 1.0)


@pytest.mark.parametrize("sink", ["exact_kv", "exact_kv_and_rows"])
@pytest.mark.parametrize("mode", ["bf16", "int8_pv"])
def test_h3_conditioning_sink_on_device(pkg, dev, sink, mode):
    """A published H3 video span that starts mid-block (row 150): the blocks
    holding conditioning rows are exact keys for every query block, and with
    exact_kv_and_rows their query rows are dense too."""
    disp = _mods(pkg)[0]
    N, H, block, tau, start = 1300, 2, 64, 1.2, 150
    print(f"[h3 sink] sink={sink} mode={mode}", flush=True)
    hq, hk, hv = _field(N, H, 31), _field(N, H, 32), _field(N, H, 33)
    q, k, v = (t.to(dev) for t in (hq, hk, hv))
    cover = (0, -(-start // block))
    sink_q = cover if sink == "exact_kv_and_rows" else (0, 0)
    direct = _direct(pkg, q, k, v, mode, tau=tau, block=block, sink_blocks=cover, sink_q=sink_q)
    ov = disp.make_override(tau=tau, min_tokens=0, block=block, sink_conditioning=sink,
                            **MODES[mode])
    flat = [t.reshape(1, N, H * 128) for t in (q, k, v)]
    out = ov(_dense([]), *flat, H, transformer_options={"sol_h3_video_span": (start, N)})
    assert torch.equal(out.view(1, N, H, 128), direct)
    plain = _direct(pkg, q, k, v, mode, tau=tau, block=block)
    assert not torch.equal(plain, direct)  # the sink changed the routing
    _against_oracle(f"h3 sink {sink} {mode}", direct, hq, hk, hv, mode, block, tau,
                    sink_kv=cover, sink_q=sink_q)


def _h3_gpu_module(H, tri):
    """A stand-in MiniMax-H3 model module on the device: PackedLayout (text,
    audio, then the patchified video rows) and a block stack whose attention is
    the sparse kernel with every block exact (tau = -inf, dense attention)."""
    mod = types.ModuleType("fake_h3_gpu_model")

    class PackedLayout:
        def __init__(self, text_len, latent_t, latent_h, latent_w, audio_t):
            video = latent_t * (latent_h // 2) * (latent_w // 2)
            cond = text_len + audio_t
            self.segments = [(0, text_len, "text"), (text_len, cond, "audio"),
                             (cond, cond + video, "video")]
            self.position_ids = torch.arange(cond + video)

    class Block(torch.nn.Module):
        def __init__(self, log):
            super().__init__()
            self.log = log

        def forward(self, h, t_emb, mod_segments, rope, extra=None):
            self.log.append(rope)
            S = h.shape[0]
            qk = (h * rope[0]).view(1, S, H, 128)
            return tri.sol_attn(qk, qk, h.view(1, S, H, 128), tau=-1e30, block=64).view(S, H * 128)

    class Model(torch.nn.Module):
        def __init__(self):
            super().__init__()
            self.seen = []
            self.blocks = torch.nn.ModuleList([Block(self.seen) for _ in range(2)])

        def rope_freqs(self, position_ids, device):
            g = torch.Generator().manual_seed(int(position_ids.numel()))
            n = position_ids.numel()
            return (torch.rand(1, n, H * 128, generator=g) + 0.5).to(torch.bfloat16).to(device)

        def _forward(self, x, timestep, context, transformer_options={}, layout_args=None):
            self.seen.clear()
            layout = sys.modules[type(self).__module__].PackedLayout(*layout_args)
            rope = self.rope_freqs(layout.position_ids, x.device)
            h = x
            for blk in self.blocks:
                h = blk(h, None, None, rope)
            return h

    mod.PackedLayout, mod.Model = PackedLayout, Model
    Model.__module__ = mod.__name__
    sys.modules[mod.__name__] = mod
    return mod


@pytest.mark.parametrize("block", [64, 128])
@pytest.mark.parametrize("text_len", [64, 37])  # span start on and off the block grid
def test_h3_hooks_through_gather_kernel(pkg, dev, block, text_len):
    """The H3 hooks on device tensors: rows and the RoPE table are gathered by
    the HIP kernel with the composed index (identity before the span, the
    rotated Morton order inside it), the blocks see the permuted table, and the
    stack's output comes back in the original order (neutral against the
    un-hooked pass, whose attention is dense)."""
    h3 = importlib.import_module(f"{pkg.__name__}._morton_h3")
    tri = _mods(pkg)[1]
    H = 2
    mod = _h3_gpu_module(H, tri)
    model = mod.Model()
    h3.install_h3_morton(model, block=64)
    layout_args = (text_len, 4, 16, 16, 10)  # video 4 x 8 x 8 = 256 rows after 10 audio rows
    start = text_len + 10
    S = start + 256
    print(f"[h3 hooks] block={block} text_len={text_len} S={S}", flush=True)
    x = (torch.randn(S, H * 128, generator=torch.Generator().manual_seed(5)) * 0.5).to(
        torch.bfloat16).to(dev)
    plain = model._forward(x, None, None, transformer_options={}, layout_args=layout_args)
    table = model.seen[0]
    opts = {"sol_morton": True, "sol_morton_curve": "3d", "sol_block_size": block}
    hooked = model._forward(x, None, None, transformer_options=opts, layout_args=layout_args)
    torch.cuda.synchronize()
    fwd, inv = h3._composed((4, 8, 8), "3d", x.device, start, S, S, block)
    assert torch.equal(fwd[:start].cpu(), torch.arange(start))
    assert torch.equal(fwd[inv].cpu(), torch.arange(S))
    assert all(torch.equal(r, table[:, fwd]) for r in model.seen)  # gathered bit for bit
    err = (hooked.float() - plain.float()).abs().max().item()
    cos = cosine(hooked.float().cpu().numpy(), plain.float().cpu().numpy())
    print(f"[h3 hooks] max |hooked - plain| = {err:.3e} cos={cos:.6f}", flush=True)
    assert err < BF16_MAXABS and cos >= BF16_COS
