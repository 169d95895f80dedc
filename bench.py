"""Benchmark of the Sol-Attn sparse attention path on one MI355X.

(placeholder: the measurement driver follows; this module already provides the
synthetic workloads shared with the tests)
"""

from __future__ import annotations

import math

import torch
import torch.nn.functional as F

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
    q = smooth_field(B, H, D, cfg["grid"], cfg["coarse"], cfg["sigma"], 0, device)
    k = smooth_field(B, H, D, cfg["grid"], cfg["coarse"], cfg["sigma"], 1, device)
    v = smooth_field(B, H, D, cfg["grid"], cfg["coarse"], cfg["sigma"], 2, device)
    if cfg.get("k_offset"):
        g = torch.Generator().manual_seed(3)
        k = k + (cfg["k_offset"] * torch.randn(1, 1, H, D, generator=g)).to(device)
    if dtype is None:
        dtype = torch.float32 if cfg["dtype"] == "fp32" else torch.bfloat16
    return q.to(dtype), k.to(dtype), v.to(dtype)
