"""Benchmark of the Sol-Attn sparse attention path on one MI355X.

Workload (the "32K tokens" of the headline metric):
B=1, H=24, D=128, N=32760 tokens from a 21x30x52 latent grid (smooth seeded
field + 0.2 N(0,1) noise), Morton 3d reordered, routing block 128, tau=0.9.

A step is one sparse-attention call (``sol_attn``: pool -> moments -> route ->
BF16 forward) on inputs already resident in HBM. Prints ONE JSON line:
value = dense-equivalent TFLOPS (4*B*H*N^2*D / time per call), ms_per_step =
ms per call, plus the roofline of the dominant kernel (the forward, timed alone
with HIP events on its stream) and the CPU baseline (the oracle's masked
attention path, timed on a bounded sample on this host).

    python bench.py [--steps K] [--warmup W] [--config 2] [--no-cpu] [--extra]
"""

from __future__ import annotations

import argparse
import importlib
import json
import math
import os
import sys
import time

import torch
import torch.nn.functional as F

ROOT = os.path.dirname(os.path.abspath(__file__))

# Workloads of BASELINE.json. grid = latent (T, H, W); coarse = seeded grid
# that is trilinearly upsampled into a smooth field; sigma = noise level.
CONFIGS = {
    0: dict(name="cpu_plumbing", B=1, H=4, D=64, grid=(4, 32, 32), coarse=(2, 8, 8), sigma=0.3,
            block=64, tau=0.9, dtype="fp32", morton=True, k_offset=0.0),
    1: dict(name="image_dit", B=1, H=24, D=128, grid=(1, 64, 64), coarse=(2, 8, 8), sigma=0.3,
            block=64, tau=0.9, dtype="bf16", morton=False, k_offset=0.5),
    2: dict(name="video_32k", B=1, H=24, D=128, grid=(21, 30, 52), coarse=(4, 6, 8), sigma=0.2,
            block=128, tau=0.9, dtype="bf16", morton=True, k_offset=0.0),
    3: dict(name="video_32k_int8", B=1, H=24, D=128, grid=(21, 30, 52), coarse=(4, 6, 8), sigma=0.2,
            block=128, tau=0.9, dtype="bf16", morton=True, k_offset=0.0, int8=True),
    4: dict(name="long_video_75k", B=1, H=40, D=128, grid=(21, 60, 60), coarse=(4, 8, 8), sigma=0.2,
            block=128, tau=0.9, dtype="bf16", morton=True, k_offset=0.0),
}

PEAK_BF16_TFLOPS = 2500.0   # MI355X dense bf16 MFMA
PEAK_INT8_TOPS = 5000.0     # MI355X dense int8 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E


def smooth_field(B, H, D, grid, coarse, sigma, seed, device="cpu"):
    """[B, N, H, D] float32: a seeded coarse N(0,1) grid trilinearly upsampled to
    ``grid`` (raster t, h, w order) plus sigma * N(0,1) noise."""
    g = torch.Generator().manual_seed(seed)
    c = torch.randn(B, H * D, *coarse, generator=g)
    noise = torch.randn(B, math.prod(grid), H, D, generator=g)
    c = c.to(device)
    f = F.interpolate(c, size=tuple(grid), mode="trilinear", align_corners=True)
    f = f.reshape(B, H * D, -1).transpose(1, 2).reshape(B, -1, H, D)
    return f + sigma * noise.to(device)


def make_inputs(cfg, device="cpu", dtype=None):
    """(q, k, v) for a config dict (seeds 0, 1, 2), cast to the config's dtype."""
    B, H, D = cfg["B"], cfg["H"], cfg["D"]
    if dtype is None:
        dtype = torch.float32 if cfg["dtype"] == "fp32" else torch.bfloat16
    out = []
    for seed in (0, 1, 2):
        t = smooth_field(B, H, D, cfg["grid"], cfg["coarse"], cfg["sigma"], seed, device)
        if seed == 1 and cfg.get("k_offset"):
            g = torch.Generator().manual_seed(3)
            t = t + (cfg["k_offset"] * torch.randn(1, 1, H, D, generator=g)).to(device)
        out.append(t.to(dtype).contiguous())
        del t
    return tuple(out)


def dense_flops(B, H, N, D):
    return 4.0 * B * H * N * N * D


def routed_flops(counts, mask, T, block, D):
    """Algorithmic FLOPs of the forward on valid tokens:
    4*D*sum_{b,h,i} len_i * (sum_{j exact} len_j + |approx(i)|)."""
    NT = (T + block - 1) // block
    lens = torch.full((NT,), float(block), dtype=torch.float64)
    lens[-1] = T - (NT - 1) * block
    j = torch.arange(NT)
    words = mask.to(torch.int64)[..., j >> 5] & 0xFFFFFFFF
    ex = ((words >> (j & 31)) & 1).bool()  # [B,H,NT,NT]
    exact_tok = (ex.double() * lens).sum(-1)
    n_approx = (~ex).sum(-1).double()
    return float(4 * D * (lens * (exact_tok + n_approx)).sum())


def split_ops(counts, mask, T, block, D):
    """(exact, pooled) algorithmic ops of the forward on valid tokens: half of
    each is QK, half P.V (the terms of routed_flops)."""
    NT = (T + block - 1) // block
    lens = torch.full((NT,), float(block), dtype=torch.float64)
    lens[-1] = T - (NT - 1) * block
    j = torch.arange(NT)
    words = mask.to(torch.int64)[..., j >> 5] & 0xFFFFFFFF
    ex = ((words >> (j & 31)) & 1).bool()
    exact = float(4 * D * (lens * (ex.double() * lens).sum(-1)).sum())
    pooled = float(4 * D * (lens * (~ex).sum(-1).double()).sum())
    return exact, pooled


def int8_roofline(ms, exact, pooled, int8_pv):
    """Fraction of the MFMA roofline for the INT8 forward: the time the op mix
    takes at peak (QK on int8 MFMA, exact P.V on int8 or bf16 MFMA, pooled tiles
    on bf16 MFMA) over the measured launch time."""
    ideal_ms = 1e3 * (exact / 2 / (PEAK_INT8_TOPS * 1e12)
                      + exact / 2 / ((PEAK_INT8_TOPS if int8_pv else PEAK_BF16_TFLOPS) * 1e12)
                      + pooled / (PEAK_BF16_TFLOPS * 1e12))
    return {"launch_ms": round(ms, 4), "exact_ops": exact, "pooled_flops": pooled,
            "ideal_ms_at_peak": round(ideal_ms, 4), "frac": round(ideal_ms / ms, 4),
            "tops": round((exact + pooled) / (ms * 1e-3) / 1e12, 2)}


def time_cuda(fn, steps, warmup):
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    start, end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    start.record()
    for _ in range(steps):
        fn()
    end.record()
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def _pkg():
    sys.path.insert(0, ROOT)
    from __graft_entry__ import PKG_NAME, load_package
    import importlib

    load_package()
    return {m: importlib.import_module(f"{PKG_NAME}.{m}")
            for m in ("_tri_fwd", "_int8_fwd", "_preprocess", "_fused_prep", "_morton")}


def torch_sdpa(q, k, v, dflops, steps):
    """PyTorch's dense SDPA at the same shape (the path ComfyUI takes when the
    node declines): BHND contiguous bf16, fused backends only (flash, then
    memory-efficient); a backend that has no kernel for this GPU raises and is
    recorded instead of falling back to the unfused math path."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    qh, kh, vh = (t.transpose(1, 2).contiguous() for t in (q, k, v))
    tried = {}
    for name, backend in (("flash", SDPBackend.FLASH_ATTENTION),
                          ("efficient", SDPBackend.EFFICIENT_ATTENTION)):
        try:
            with sdpa_kernel([backend]):
                ms = time_cuda(lambda: F.scaled_dot_product_attention(qh, kh, vh), steps, 1)
            return {"backend": name, "ms": round(ms, 3),
                    "dense_tflops": round(dflops / (ms * 1e-3) / 1e12, 1), "unavailable": tried}
        except RuntimeError as e:
            tried[name] = str(e).splitlines()[0][:160]
    return {"backend": None, "unavailable": tried}


def cpu_baseline(cfg, q, k, v, budget_s=15.0):
    """The oracle's masked-attention CPU path (torch fp32, augmented keys, one
    query block at a time) on a bounded sample of query blocks; the oracle's C
    routing runs on the full input. Extrapolated to ms per call."""
    sys.path.insert(0, ROOT)
    import numpy as np
    import oracle  # test infrastructure: the CPU baseline leg only

    threads = torch.get_num_threads()
    bits = lambda t: t.contiguous().cpu().view(torch.int16).numpy().view(np.uint16)
    qb, kb, vb = bits(q), bits(k), bits(v)
    t0 = time.perf_counter()
    prep = oracle.prepare(qb, kb, vb, block=cfg["block"], tau=cfg["tau"])
    t_prep = time.perf_counter() - t0
    B, T, H, D = q.shape
    NT = prep["NT"]
    qf, kf, vf = (t.float().cpu() for t in (q, k, v))
    rng = np.random.default_rng(0)
    order = [(h, i) for h in range(H) for i in range(NT)]
    rng.shuffle(order)
    done, t_attn = 0, 0.0
    while done < len(order) and t_attn < budget_s:
        h, i = order[done]
        t1 = time.perf_counter()
        oracle.masked_attention_torch(qf, kf, vf, prep, heads=[h], qblocks=[i])
        t_attn += time.perf_counter() - t1
        done += 1
    per_call_s = t_prep + t_attn * (len(order) / done)
    return {
        "value": round(per_call_s * 1e3, 1),
        "unit": "ms/call",
        "cores": threads,
        "kind": "port",
        "cpu": _cpu_model(),
        "sample": (f"reference semantics, restated (the reference has no CPU path): oracle C "
                   f"routing on the full input ({t_prep:.2f} s) + torch-fp32 masked attention "
                   f"over [tokens; pooled keys] for {done} of {len(order)} (head, query-block) "
                   f"pairs ({t_attn:.1f} s), scaled to the full call"),
        "dense_equiv_tflops": round(dense_flops(B, H, T, D) / per_call_s / 1e12, 4),
    }


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip() + f" ({os.cpu_count()} logical CPUs)"
    except OSError:
        pass
    return None


def _traffic():
    """HBM bytes per forward launch from the committed rocprofv3 --pmc summary."""
    path = os.path.join(ROOT, "profiles", "fwd_bf16_video32k_traffic.json")
    try:
        with open(path) as f:
            return json.load(f).get("bytes_per_launch")
    except (OSError, ValueError):
        return None


def run_kernel_only(args, mods, cfg, q, k, v):
    """Launch one kernel ``--steps`` times for rocprofv3 (kernel trace or --pmc
    passes), preceded by a 512 MiB copy whose bytes are known exactly."""
    block, tau, D = cfg["block"], cfg["tau"], q.shape[-1]
    src = torch.empty(256 << 20, dtype=torch.int16, device=q.device)
    dst = torch.empty_like(src)
    dst.copy_(src)  # calibration: 512 MiB read + 512 MiB written
    torch.cuda.synchronize()
    del src, dst
    if args.kernel_only == "fwd":
        r = mods["_preprocess"].route(q, k, v, scale=D ** -0.5, tau=tau, block=block)
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        for _ in range(args.steps):
            mods["_tri_fwd"].forward_bf16(q, k, v, r, out=out)
    elif args.kernel_only in ("fwd_int8", "fwd_int8_bf16pv", "fwd_int8_run"):
        fp = mods["_fused_prep"].fused_preprocess_routing(q, k, v, tau=tau, scale=D ** -0.5,
                                                          block=block)
        r, qi, qs, ki, ks, vi = fp
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        pv = args.kernel_only != "fwd_int8_bf16pv"
        codes = "running" if args.kernel_only == "fwd_int8_run" else "block"
        for _ in range(args.steps):
            mods["_int8_fwd"].forward_int8(q, v, r, qi, qs, ki, ks, vi, int8_pv=pv, out=out,
                                           pv_codes=codes)
    elif args.kernel_only == "quant":
        fq = importlib.import_module(mods["_preprocess"].__name__.rsplit(".", 1)[0] + "._fused_quant")
        fp = mods["_fused_prep"].fused_preprocess_routing(q, k, v, tau=tau, scale=D ** -0.5,
                                                          block=block)
        r = fp[0]
        for _ in range(args.steps):
            fq.quantize_bthd(q)
            fq.quantize_bthd(k, mean=r.kc_mean.reshape(-1, D))
            fq.quantize_v_per_channel(v)
    elif args.kernel_only in ("int8_call", "int8_bf16pv_call", "int8_run_call"):
        pv = args.kernel_only != "int8_bf16pv_call"
        codes = "running" if args.kernel_only == "int8_run_call" else "block"
        for _ in range(args.steps):
            mods["_int8_fwd"].sol_attn_int8(q, k, v, tau=tau, block=block, int8_pv=pv,
                                            pv_codes=codes)
    elif args.kernel_only == "bf16_call":
        for _ in range(args.steps):
            mods["_tri_fwd"].sol_attn(q, k, v, tau=tau, block=block)
    elif args.kernel_only == "prep":
        for _ in range(args.steps):
            mods["_preprocess"].route(q, k, v, scale=D ** -0.5, tau=tau, block=block)
    else:
        perm, _ = mods["_morton"].morton_perm(cfg["grid"], q.device, "3d")
        for _ in range(args.steps):
            mods["_morton"].reorder_tokens(q, perm, dim=1)
    torch.cuda.synchronize()
    print(f"[bench] kernel-only {args.kernel_only} x{args.steps} done", file=sys.stderr, flush=True)


# Sequence lengths for the dense/sparse crossover (the node's min_tokens):
# video-like smooth fields on latent grids of these token counts.
SWEEP_GRIDS = [(1, 32, 32), (2, 32, 32), (4, 32, 32), (8, 32, 32), (16, 32, 32), (21, 30, 52)]
SWEEP_TAUS = (0.8, 0.9, 1.3)


def run_sweep(args, mods, dev):
    """Dense PyTorch SDPA (the path the node declines to) against the sparse
    calls (prep included) per sequence length and tau, at both block sizes:
    one JSON line per (N, block). Morton reordering is per model, not per
    call, so it is done before timing."""
    sol_attn = mods["_tri_fwd"].sol_attn
    i8 = mods["_int8_fwd"].sol_attn_int8
    steps = max(3, args.steps // 2)
    for grid in SWEEP_GRIDS:
        cfg = dict(CONFIGS[2], grid=grid, coarse=(min(4, grid[0]), 6, 8))
        q, k, v = make_inputs(cfg, dev)
        perm, _ = mods["_morton"].morton_perm(grid, dev, "3d")
        q, k, v = (mods["_morton"].reorder_tokens(t, perm, dim=1) for t in (q, k, v))
        B, T, H, D = q.shape
        dflops = dense_flops(B, H, T, D)
        sdpa = torch_sdpa(q, k, v, dflops, steps)
        for block in (64, 128):
            line = {"N": T, "H": H, "block": block, "sdpa_ms": sdpa.get("ms"),
                    "sdpa_backend": sdpa.get("backend"), "bf16_ms": {}, "int8_pv_ms": {},
                    "int8_pv_run_ms": {}, "int8_bf16pv_ms": {}, "density": {}}
            for tau in SWEEP_TAUS:
                line["bf16_ms"][str(tau)] = round(time_cuda(
                    lambda: sol_attn(q, k, v, tau=tau, block=block), steps, 2), 4)
                line["int8_pv_ms"][str(tau)] = round(time_cuda(
                    lambda: i8(q, k, v, tau=tau, block=block, int8_pv=True), steps, 2), 4)
                line["int8_pv_run_ms"][str(tau)] = round(time_cuda(
                    lambda: i8(q, k, v, tau=tau, block=block, pv_codes="running"), steps, 2), 4)
                line["int8_bf16pv_ms"][str(tau)] = round(time_cuda(
                    lambda: i8(q, k, v, tau=tau, block=block, int8_pv=False), steps, 2), 4)
                r = mods["_preprocess"].route(q, k, v, scale=D ** -0.5, tau=tau, block=block)
                NT = r.counts.shape[-1]
                line["density"][str(tau)] = round(float(r.counts.double().sum() / (B * H * NT * NT)), 4)
            print(json.dumps(line), flush=True)
        del q, k, v
        torch.cuda.empty_cache()


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=3)
    ap.add_argument("--config", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-budget", type=float, default=15.0)
    ap.add_argument("--extra", action="store_true", help="also time the INT8 forward (cfg 3)")
    ap.add_argument("--sweep", action="store_true",
                    help="dense SDPA vs the sparse calls over sequence lengths and tau (the "
                         "min_tokens crossover); JSON lines, not the metric")
    ap.add_argument("--block", type=int, choices=[64, 128],
                    help="routing block size instead of the config's (a diagnostic, not the metric)")
    ap.add_argument("--heads", type=int,
                    help="number of heads instead of the config's, e.g. 3 = one GPU's share of an "
                         "8-way head split at cfg 2 (not the metric)")
    ap.add_argument("--kernel-only", choices=["fwd", "fwd_int8", "fwd_int8_bf16pv", "fwd_int8_run",
                                              "prep", "quant", "reorder", "int8_call",
                                              "int8_bf16pv_call", "int8_run_call", "bf16_call"],
                    help="profiling driver: run only this kernel --steps times (after a "
                         "512 MiB device copy used to calibrate memory counters); no JSON")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU: this build has no multi-GPU path "
              "(heads shard with no communication; see the sharding notes).", file=sys.stderr)
        sys.exit(2)
    if not torch.cuda.is_available():
        print("bench.py needs a HIP device", file=sys.stderr)
        sys.exit(2)

    mods = _pkg()
    dev = torch.device("cuda:0")
    if args.sweep:
        run_sweep(args, mods, dev)
        return
    cfg = dict(CONFIGS[args.config])
    if args.block:
        cfg["block"] = args.block
    if args.heads:
        cfg["H"] = args.heads
    print(f"[bench] config {args.config} {cfg['name']}: generating inputs", file=sys.stderr, flush=True)
    q, k, v = make_inputs(cfg, dev)
    B, T, H, D = q.shape
    block, tau = cfg["block"], cfg["tau"]
    reorder_ms = None
    if cfg["morton"]:
        perm, inv = mods["_morton"].morton_perm(cfg["grid"], dev, "3d")
        q, k, v = (mods["_morton"].reorder_tokens(t, perm, dim=1) for t in (q, k, v))
        reorder_ms = time_cuda(lambda: mods["_morton"].reorder_tokens(q, perm, dim=1), 10, 2)
    torch.cuda.synchronize()

    if args.kernel_only:
        run_kernel_only(args, mods, cfg, q, k, v)
        return

    sol_attn = mods["_tri_fwd"].sol_attn
    step = lambda: sol_attn(q, k, v, tau=tau, block=block)
    print("[bench] timing sol_attn", file=sys.stderr, flush=True)
    ms = time_cuda(step, args.steps, args.warmup)

    r = mods["_preprocess"].route(q, k, v, scale=D ** -0.5, tau=tau, block=block)
    out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
    fwd = lambda: mods["_tri_fwd"].forward_bf16(q, k, v, r, out=out)
    fwd_ms = time_cuda(fwd, args.steps, args.warmup)
    prep_ms = time_cuda(lambda: mods["_preprocess"].route(q, k, v, scale=D ** -0.5, tau=tau,
                                                          block=block), args.steps, args.warmup)
    counts = r.counts.cpu()
    NT = counts.shape[-1]
    density = float(counts.double().sum() / (B * H * NT * NT))
    rflops = routed_flops(counts, r.mask.cpu(), T, block, D)
    dflops = dense_flops(B, H, T, D)
    achieved = rflops / (fwd_ms * 1e-3) / 1e12
    line = {
        "metric": "ms/attention call + dense-equiv TFLOPS at 32K tokens, % of MFMA peak",
        "value": round(dflops / (ms * 1e-3) / 1e12, 2),
        "unit": "TFLOPS (dense-equivalent, one sparse attention call)",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic (seeded smooth field + noise" + (", Morton 3d reordered)" if cfg["morton"] else ")"),
        "config": {"workload": f"cfg{args.config} {cfg['name']}: B{B} H{H} D{D} N{T} grid "
                               f"{'x'.join(map(str, cfg['grid']))} block {block} tau {tau}",
                   "global_batch": B, "seq_len": T, "parallelism": "none (1 GPU)"},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_BF16_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(achieved / PEAK_BF16_TFLOPS, 4),
                     "traffic": _traffic() if (args.config, block, H) == (2, 128, 24) else None,
                     "traffic_source": ("profiles/fwd_bf16_video32k_traffic.json: rocprofv3 "
                                        "FETCH_SIZE + WRITE_SIZE of this kernel, calibrated on "
                                        "a 512 MiB copy (not measured by this run)")
                     if (args.config, block, H) == (2, 128, 24) else None,
                     "kernel": ("bf16fwd::fwd_bf16_kernel<128>" if block == 128
                                else "bf16fwd::fwd_bf16_sbuf_kernel<64>"),
                     "algorithmic_flops_per_launch": rflops, "launch_ms": round(fwd_ms, 4)},
        "routed_density": round(density, 4),
        "prep_ms": round(prep_ms, 4),
        "fwd_ms": round(fwd_ms, 4),
        "dense_equiv_tflops_fwd_only": round(dflops / (fwd_ms * 1e-3) / 1e12, 2),
        "reorder_ms_per_tensor": None if reorder_ms is None else round(reorder_ms, 4),
        "reorder_GBps": None if reorder_ms is None else round(2 * q.numel() * 2 / (reorder_ms * 1e-3) / 1e9, 1),
    }
    del r, out
    if args.extra:
        i8 = mods["_int8_fwd"].sol_attn_int8
        # int8 QK, bf16 P.V; the reference's default int8 P.V beside it
        # (_run: int8 P.V with codes against the running max, SOLATTN_PV_INT8_RUNNING)
        for key, pv, codes in (("int8_ms", False, "block"), ("int8_pv_ms", True, "block"),
                               ("int8_pv_run_ms", True, "running")):
            line[key] = {str(t): round(time_cuda(lambda: i8(q, k, v, tau=t, block=block, int8_pv=pv,
                                                            pv_codes=codes),
                                                 args.steps, args.warmup), 4) for t in (0.8, 0.9, 0.95)}
        # config 3's wording, Q/K scales per 128-token block (not the parity mode)
        for key, pv, codes in (("int8_qblock_ms", False, "block"), ("int8_pv_qblock_ms", True, "block"),
                               ("int8_pv_run_qblock_ms", True, "running")):
            line[key] = {str(t): round(time_cuda(lambda: i8(q, k, v, tau=t, block=block, int8_pv=pv,
                                                            quant_block=128, pv_codes=codes),
                                                 args.steps, args.warmup), 4) for t in (0.8, 0.9, 0.95)}
        # the INT8 forward kernel alone at the config's tau, against the MFMA roofline
        fp = mods["_fused_prep"].fused_preprocess_routing(q, k, v, tau=tau, scale=D ** -0.5,
                                                          block=block)
        ri, qi, qs, ki, ks, vi = fp
        exact, pooled = split_ops(ri.counts.cpu(), ri.mask.cpu(), T, block, D)
        out = torch.empty(q.shape, dtype=q.dtype, device=q.device)
        line["int8_fwd"] = {}
        for key, pv, codes in (("pv_bf16", False, "block"), ("pv_int8", True, "block"),
                               ("pv_int8_run", True, "running")):
            ms_i8 = time_cuda(lambda: mods["_int8_fwd"].forward_int8(q, v, ri, qi, qs, ki, ks, vi,
                                                                     int8_pv=pv, out=out,
                                                                     pv_codes=codes),
                              args.steps, args.warmup)
            line["int8_fwd"][key] = int8_roofline(ms_i8, exact, pooled, pv)
        line["int8_fwd"]["routed_density"] = round(float(ri.counts.double().sum()
                                                         / (B * H * NT * NT)), 4)
        del fp, ri, qi, qs, ki, ks, vi, out
        # dense comparator at the same shape: every block exact (tau = -inf)
        dense_ms = time_cuda(lambda: sol_attn(q, k, v, tau=-1e30, block=block), max(3, args.steps // 4),
                             1)
        line["dense_all_exact_ms"] = round(dense_ms, 3)
        line["dense_all_exact_tflops"] = round(dflops / (dense_ms * 1e-3) / 1e12, 1)
        # the sparse BF16 call per tau, beside the dense path the node falls back to
        line["bf16_ms"] = {str(t): round(time_cuda(lambda: sol_attn(q, k, v, tau=t, block=block),
                                                   args.steps, args.warmup), 4)
                           for t in (0.8, 0.9, 0.95)}
        line["torch_sdpa"] = torch_sdpa(q, k, v, dflops, max(3, args.steps // 4))
        if cfg["morton"]:
            # the whole node path on raster-order tokens: reorder q, k, v -> prep (+ quant)
            # -> sparse forward -> inverse reorder of o (BASELINE config 4's pipeline)
            mo = mods["_morton"]

            def pipeline(fn):
                qq, kk, vv = (mo.reorder_tokens(t, perm, dim=1) for t in (q, k, v))
                return mo.reorder_tokens(fn(qq, kk, vv), inv, dim=1)

            line["pipeline_ms"] = {
                "bf16": round(time_cuda(lambda: pipeline(lambda a, b, c: sol_attn(a, b, c, tau=tau, block=block)),
                                        args.steps, args.warmup), 4),
                "int8_pv": round(time_cuda(lambda: pipeline(lambda a, b, c: i8(a, b, c, tau=tau, block=block)),
                                           args.steps, args.warmup), 4),
            }
    if not args.no_cpu:
        print("[bench] CPU baseline", file=sys.stderr, flush=True)
        line["cpu_baseline"] = cpu_baseline(cfg, q, k, v, args.cpu_budget)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
