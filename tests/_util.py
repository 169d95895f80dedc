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


def mask_bits(mask_u32: np.ndarray, NT: int) -> np.ndarray:
    """Routing bitmask [..., W] uint32 -> bool [..., NT] (bit j%32 of word j/32)."""
    bits_ = (mask_u32[..., :, None] >> np.arange(32, dtype=np.uint32)) & 1
    return bits_.reshape(*mask_u32.shape[:-1], -1)[..., :NT].astype(bool)


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


# INT8 forward bounds, per query block: cosine against the reference loop's
# arithmetic (north_star's INT8 tolerance), and max-abs / cosine against the
# kernel's own documented arithmetic (RNE P codes, code-sum denominator).
INT8_COS = 0.999
INT8_KERNEL_MAXABS = 1e-2  # measured at most 2.4e-3 over the GPU cases
INT8_KERNEL_COS = 0.9995


def per_block(got: np.ndarray, ref: dict, block: int):
    """[(key, max-abs, cosine)] for each oracle query block {(b,h,i): [len, D]}
    against the full output got [B, T, H, D]."""
    stats = []
    for (b, h, i), o in ref.items():
        g = got[b, i * block:i * block + o.shape[0], h].astype(np.float64)
        stats.append(((b, h, i), float(np.abs(g - o).max()), cosine(g, o)))
    return stats


def check_int8_blocks(label, got, qb, vb, prep, rows, int8_pv, block,
                      kernel_maxabs=INT8_KERNEL_MAXABS, pv_codes="block"):
    """Per-query-block INT8 checks against the oracle's two arithmetics (the
    reference's, and the kernel's: block-max codes, or running-max codes with
    pv_codes="running"), with the worst block of each printed."""
    import oracle

    ref = oracle.forward_int8_port(qb, vb, prep, rows, int8_pv=int8_pv)
    codes = "running" if pv_codes == "running" else "kernel"
    ker = oracle.forward_int8_port(qb, vb, prep, rows, int8_pv=int8_pv, codes=codes) \
        if int8_pv else ref
    s_ref, s_ker = per_block(got, ref, block), per_block(got, ker, block)
    w_ref = min(s_ref, key=lambda s: s[2])
    w_abs = max(s_ker, key=lambda s: s[1])
    w_cos = min(s_ker, key=lambda s: s[2])
    print(f"[{label}] {len(rows)} query blocks; vs reference arithmetic: worst cos "
          f"{w_ref[2]:.6f} at {w_ref[0]} (max|err| {max(s[1] for s in s_ref):.3e}); vs kernel "
          f"arithmetic: worst max|err| {w_abs[1]:.3e} at {w_abs[0]}, worst cos {w_cos[2]:.6f} "
          f"at {w_cos[0]}", flush=True)
    assert w_ref[2] >= INT8_COS, w_ref
    assert w_abs[1] <= kernel_maxabs, w_abs
    assert w_cos[2] >= INT8_KERNEL_COS, w_cos
