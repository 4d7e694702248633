"""A CPU model of the fused stage 1's operand roundings, for its ddO epilogue
and its row statistic B.

The fused stage 1 (flash-hog_amd/csrc/fhog_bwdbwd_fused.hip) accumulates
ddO = sum_j P ddV + sum_j x V - dD O in one sweep, x = P ddS, where the
matrix products take P and x rounded to bf16. When a row's keys carry similar
x, sum_j x V - dD O cancels to sum_j x (V_j - O), and the rounding of x leaves
a residue unless the subtracted dD is the sum of the same rounded x. This
model reproduces the kernel's roundings in float64 numpy (bf16 operands,
fp32-exact products) on a problem whose rows see few keys, and shows that the
rounded dD halves the ddO error against the fp64 oracle (the GPU sweep,
tests/test_gpu_sweep.py p74, runs the same inputs through the kernel). CPU only.
"""

from __future__ import annotations

import numpy as np
import torch

from helpers import make_inputs, to_np
from oracle import attention as ora


def _bf16(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.bfloat16).double().numpy()


def _ddo_errors(B, Nq, Nk, H, Hk, D, causal, seed):
    scale = D ** -0.5
    x = make_inputs(B, Nq, Nk, H, D, torch.bfloat16, seed=seed, kv_heads=Hk)
    o_ref, lse = ora.attn_fwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), scale, causal)
    o = _bf16(o_ref)
    lse = lse.astype(np.float32).astype(np.float64)
    ref = ora.attn_bwd_bwd_stats(*(to_np(x[n]) for n in ("q", "k", "v")), o, to_np(x["do"]),
                                 *(to_np(x[n]) for n in ("ddq", "ddk", "ddv")), lse, scale, causal)
    ddo_ref = ref[3]
    errs = {}
    for rounded in (False, True):
        ddo = np.zeros_like(ddo_ref)
        for b in range(B):
            for h in range(H):
                hk = h // (H // Hk)
                q, ddq = to_np(x["q"])[b, :, h], to_np(x["ddq"])[b, :, h]
                k, v, ddk, ddv = (to_np(x[n])[b, :, hk] for n in ("k", "v", "ddk", "ddv"))
                mask = np.arange(Nk)[None, :] <= np.arange(Nq)[:, None]  # top-left causal
                p = np.where(mask, np.exp(scale * q @ k.T - lse[b, h][:, None]), 0.0)
                xs = p * scale * (ddq @ k.T + q @ ddk.T)
                acc = _bf16(p) @ ddv + _bf16(xs) @ v
                dd = (_bf16(xs) if rounded else xs).sum(-1)
                ddo[b, :, h] = acc - dd[:, None] * o[b, :, h]
        errs[rounded] = float(np.abs(ddo - ddo_ref).max() / np.abs(ddo_ref).max())
    return errs


def test_rounded_dd_halves_the_ddo_error_where_rows_see_few_keys():
    # the inputs of tests/test_gpu_sweep.py p74: B2, N_Q 298, N_K 34, 2 query heads on 1 key/value head
    errs = _ddo_errors(2, 298, 34, 2, 1, 64, causal=1, seed=101 + 74)
    assert errs[False] > 1.5e-2, errs  # the unrounded dD: at the bf16 tolerance
    assert errs[True] < 1e-2, errs     # the kernel's rounded dD
    assert errs[True] < 0.6 * errs[False], errs


def test_b_statistic_error_is_at_the_scale_of_c():
    """The fused stage 1 forms the row statistic B as c - D dD with
    c = <dO, ddO>, ddO accumulated from P and P ddS rounded to bf16. On the
    problem of tests/test_gpu_sweep.py s31p07 (one query row, N_K 78, D 128,
    scale 0.1247), c = 0.284 and D dD = 0.269 nearly cancel: the model's B is
    far off relative to B (which is why tests/helpers.py b_stat_err measures
    it against |c|), and within 1e-2 of |c|, the scale at which pass 4 uses it
    (dS2 = P (dP2 - B), flash_hog/jax/_pallas_gpu_kernel.py:358)."""
    B, Nq, Nk, H, D, scale = 1, 1, 78, 1, 128, 0.1247
    x = make_inputs(B, Nq, Nk, H, D, torch.bfloat16, seed=108)
    o_ref, lse = ora.attn_fwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), scale, 0)
    o = _bf16(o_ref)
    lse = lse.astype(np.float32).astype(np.float64)
    ref = ora.attn_bwd_bwd_stats(*(to_np(x[n]) for n in ("q", "k", "v")), o, to_np(x["do"]),
                                 *(to_np(x[n]) for n in ("ddq", "ddk", "ddv")), lse, scale, 0, return_stats=True)
    d_ref, dd_ref, b_ref = (float(r[0, 0, 0]) for r in ref[4:])
    q, do, ddq, k, v, ddk, ddv = (to_np(x[n])[0, :, 0] for n in ("q", "do", "ddq", "k", "v", "ddk", "ddv"))
    p = np.exp(scale * q @ k.T - lse[0, 0][:, None])
    xs = p * scale * (ddq @ k.T + q @ ddk.T)
    d = float((o[0, :, 0] * do).sum())
    dd = float(xs.sum())
    ddo = _bf16(p) @ ddv + _bf16(xs) @ v - _bf16(xs).sum(-1)[:, None] * o[0, :, 0]
    b_model = float((do * ddo).sum()) - d * dd
    c_ref = d_ref * dd_ref + b_ref
    assert abs(c_ref) > 10 * abs(b_ref)
    assert abs(b_model - b_ref) > 0.1 * abs(b_ref)
    assert abs(b_model - b_ref) < 1e-2 * abs(c_ref)
