"""Helpers shared by the tests: bf16 bit views, comparisons, small cases."""

import numpy as np
import torch


def bits(t: torch.Tensor) -> np.ndarray:
    """bf16 tensor (any device) -> contiguous uint16 numpy bit patterns."""
    return t.detach().contiguous().cpu().view(torch.int16).numpy().view(np.uint16)


def from_bits(a: np.ndarray, device="cpu") -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a).view(np.int16)).view(torch.bfloat16).to(device)


def u32(t: torch.Tensor) -> np.ndarray:
    return t.detach().cpu().numpy().view(np.uint32)


def cosine(a, b) -> float:
    a = np.asarray(a, np.float64).ravel()
    b = np.asarray(b, np.float64).ravel()
    return float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-300))


def randn_bf16(shape, seed, scale=1.0):
    g = torch.Generator().manual_seed(seed)
    return (torch.randn(*shape, generator=g) * scale).to(torch.bfloat16)


def compare_rows(got: np.ndarray, ref: dict, block: int):
    """max-abs error and cosine between a full output [B,T,H,D] and oracle rows."""
    errs, g_all, r_all = [], [], []
    for (b, h, i), o in ref.items():
        lo = i * block
        g = got[b, lo:lo + o.shape[0], h].astype(np.float64)
        errs.append(np.abs(g - o).max())
        g_all.append(g.ravel())
        r_all.append(np.asarray(o, np.float64).ravel())
    return float(max(errs)), cosine(np.concatenate(g_all), np.concatenate(r_all))
