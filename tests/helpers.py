"""Shared input generation and comparison helpers for the test suite."""

from __future__ import annotations

import math

import numpy as np
import torch

# Per-output tolerance on max|a - r| / max|r| (the parity bar of this path):
# fp32 runs below 1e-3; bf16/fp16 runs below 2e-2 against an fp32-or-better reference.
TOL = {torch.float32: 1e-3, torch.float16: 2e-2, torch.bfloat16: 2e-2}

# Order in which per-tensor seeds are derived: seed + index.
TENSOR_ORDER = ("q", "k", "v", "do", "ddq", "ddk", "ddv")


def make_inputs(batch, n_q, n_k, heads, head_dim, dtype, seed=0, qkv_scale=1.0, device="cpu", kv_heads=None):
    """Seeded N(0, 1) inputs in (B, T, N, H) layout, rounded to dtype.

    Tensor i of TENSOR_ORDER is drawn from torch.Generator seeded with seed + i;
    q, k, v are multiplied by qkv_scale before rounding. k, v, ddk, ddv have
    kv_heads heads (default: heads).
    """
    kv_heads = heads if kv_heads is None else kv_heads
    shapes = {"q": (batch, n_q, heads, head_dim), "do": (batch, n_q, heads, head_dim),
              "ddq": (batch, n_q, heads, head_dim)}
    out = {}
    for i, name in enumerate(TENSOR_ORDER):
        shape = shapes.get(name, (batch, n_k, kv_heads, head_dim))
        gen = torch.Generator().manual_seed(seed + i)
        x = torch.randn(shape, generator=gen, dtype=torch.float32)
        if name in ("q", "k", "v"):
            x = x * qkv_scale
        out[name] = x.to(dtype).to(device)
    return out


def rel_err(a, r, floor: float = 0.0) -> float:
    """max|a - r| / max(max|r|, floor).

    floor keeps outputs that are identically zero in exact arithmetic (for
    example dQ of a single-token sequence, where P = 1 and dP = D) from being
    divided by round-off: their error is then measured against floor.
    """
    a = torch.as_tensor(a).double().cpu()
    r = torch.as_tensor(r).double().cpu()
    den = max(r.abs().max().item() if r.numel() else 0.0, floor)
    num = (a - r).abs().max().item() if r.numel() else 0.0
    return num / den if den > 0 else num


# Output magnitudes of the seeded N(0, 1) problems are O(1); a reference whose
# largest entry is below this is treated as exactly zero (see rel_err).
DEGENERATE_FLOOR = 1e-2


def b_stat_err(b, ref_d, ref_dd, ref_b) -> float:
    """Error of the double backward's row statistic B on the scale it is used at.

    B is scratch between the passes (TkBwdBwd returns it as such,
    flash_hog/csrc/tk_bwdbwd/ffi.cu:79-98): pass 4 uses it only in
    dS2 = P (dP2 - B) (flash_hog/jax/_pallas_gpu_kernel.py:247, 358), i.e.
    through c = D dD + B, so its error matters on the scale of c: where c
    and D dD nearly cancel, B is small, and an error the size of c's
    rounding (as in the two-sweep fp32 stage 1, B = r1 - dD r2 - D dD + r3)
    is large relative to B alone. So max|b - ref_b| is measured against
    max(max|ref_b|, max|c_ref|, floor).
    """
    b, ref_d, ref_dd, ref_b = (torch.as_tensor(t).double().cpu() for t in (b, ref_d, ref_dd, ref_b))
    c_ref = ref_d * ref_dd + ref_b
    den = max(ref_b.abs().max().item(), c_ref.abs().max().item(), DEGENERATE_FLOOR)
    return (b - ref_b).abs().max().item() / den


def stat_errs(got, ref):
    """Relative errors of the returned row statistics D, dD and B, each on its
    own scale (rel_err with the degenerate floor). b_stat_err is the looser
    measure on the scale of c = D dD + B, kept for diagnostics."""
    return tuple(rel_err(g, r, DEGENERATE_FLOOR) for g, r in zip(got[:3], ref[:3]))


def default_scale(head_dim: int) -> float:
    return 1.0 / math.sqrt(head_dim)


def to_np(t: torch.Tensor) -> np.ndarray:
    return t.detach().double().cpu().numpy()
