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
tests/test_gpu_sweep.py p74, runs the same inputs through the kernel). It also
shows why the kernel sums B from per-pair terms rather than forming it from
ddO. CPU only.
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


def _b_forms(B, Nq, Nk, H, D, causal, scale, seed):
    """The oracle's B and dK2, and per head the fused stage 1's two forms of B:
    the dot-product form <dO, ddO> - D dD with ddO accumulated from P and
    x = P ddS rounded to bf16 (the kernel's earlier form), and the per-pair
    sums sum X - dD (sum P u + D) with X = P (dPa + ddS u), u = dP - D (its
    current form); with dK2 from each B through the oracle's pass 4."""
    x = make_inputs(B, Nq, Nk, H, D, torch.bfloat16, seed=seed)
    n = {k: to_np(v) for k, v in x.items()}
    o_ref, lse = ora.attn_fwd(n["q"], n["k"], n["v"], scale, causal)
    o = _bf16(o_ref)
    lse = lse.astype(np.float32).astype(np.float64)
    ref = ora.attn_bwd_bwd_stats(n["q"], n["k"], n["v"], o, n["do"], n["ddq"], n["ddk"], n["ddv"], lse, scale,
                                 causal, return_stats=True)
    out = {"ref": (ref[6], ref[1])}
    for form in ("dot", "sums"):
        bs, dk2 = np.zeros_like(ref[6]), np.zeros_like(ref[1])
        for b in range(B):
            for h in range(H):
                q, do, ddq, k, v, ddk, ddv = (n[t][b, :, h] for t in ("q", "do", "ddq", "k", "v", "ddk", "ddv"))
                p = ora._probs(q, k, lse[b, h], scale, causal)
                dp, dpa = do @ v.T, do @ ddv.T
                dds = scale * (ddq @ k.T + q @ ddk.T)
                d = np.sum(o[b, :, h] * do, -1)
                xs = p * dds
                dd = xs.sum(-1)
                u = dp - d[:, None]
                if form == "dot":
                    ddo = _bf16(p) @ ddv + _bf16(xs) @ v - _bf16(xs).sum(-1)[:, None] * o[b, :, h]
                    bb = (do * ddo).sum(-1) - d * dd
                else:
                    bb = (p * (dpa + dds * u)).sum(-1) - dd * ((p * u).sum(-1) + d)
                dp2 = dpa - dp * dd[:, None] - dds * d[:, None] + dp * dds
                ds, ds2 = scale * p * u, scale * p * (dp2 - bb[:, None])
                bs[b, h], dk2[b, :, h] = bb, ds.T @ ddq + ds2.T @ q
        out[form] = (bs, dk2)
    out["c"] = ref[4] * ref[5] + ref[6]
    return out


def _dk2_err(dk2, ref):
    return float(np.abs(dk2 - ref).max() / np.abs(ref).max())


def test_b_statistic_from_per_pair_sums():
    """B of the fused stage 1 (flash-hog_amd/csrc/fhog_bwdbwd_fused.hip).
    On the problem of tests/test_gpu_sweep.py s31p07 (one query row, N_K 78,
    D 128, scale 0.1247) c = 0.284 and D dD = 0.269 nearly cancel: the
    dot-product form is more than 10 % off B (within 1e-2 of |c|, the scale
    at which pass 4 uses it: dS2 = P (dP2 - B),
    flash_hog/jax/_pallas_gpu_kernel.py:358). On s79p08 (four queries,
    N_K 201, D 256, bottom-right mask) its error puts dK2 over the 2e-2 bf16
    bar. The per-pair sums give the oracle's B (its definition sum P dP2,
    _pallas_gpu_kernel.py:209-210) to 1e-6 of |c| on both (sum_j P is 1 only up to
    the fp32 L), and dK2 to 1e-6."""
    s31 = _b_forms(1, 1, 78, 1, 128, 0, 0.1247, 108)
    b_ref, dk2_ref = s31["ref"]
    c = np.abs(s31["c"]).max()
    assert c > 10 * np.abs(b_ref).max()
    assert np.abs(s31["dot"][0] - b_ref).max() > 0.1 * np.abs(b_ref).max()
    assert np.abs(s31["dot"][0] - b_ref).max() < 1e-2 * c
    assert np.abs(s31["sums"][0] - b_ref).max() < 1e-6 * c  # sum_j P = 1 up to the fp32 L

    s79 = _b_forms(1, 4, 201, 3, 256, 2, 0.1843, 109)
    b_ref, dk2_ref = s79["ref"]
    assert _dk2_err(s79["dot"][1], dk2_ref) > 2e-2
    assert np.abs(s79["sums"][0] - b_ref).max() < 1e-6 * np.abs(s79["c"]).max()
    assert _dk2_err(s79["sums"][1], dk2_ref) < 1e-6
