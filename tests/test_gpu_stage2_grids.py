"""The double backward on shapes that select each of stage 2's grid layouts.

Stage 2 (pass 4, tiled over key blocks: 128 keys at D = 64 and 256, 64 keys
in the 16-key-per-wave kernel used for 2-byte types at D = 128, which keeps
plain rank-major or chunked order) lays its grid out by the problem's
size: one key block per workgroup when the grid fits on the GPU at once; for
larger causal grids a workgroup takes key block r and then its mirror
nkb - 1 - r (odd nkb leaves the middle block alone); and when that paired grid
is exactly two workgroups per CU the pairs are skewed (the standard
configuration in test_gpu_configs.py). A workgroup streams the query tiles
of both its blocks through one ring, and a block no query sees (top-left
causal with N_K > N_Q) streams nothing and writes zeros. Each shape here is
checked on every (batch, head) against tests/gpu_reference.py (fp32 closed
form on the GPU, pinned to the fp64 oracle in test_gpu_parity.py), with the
residual (O, L) from gpu_reference.fwd. Tolerance: max|a - r| / max|r| < 2e-2
(bf16 against an fp32 reference).
"""

from __future__ import annotations

import math

import pytest
import torch

import gpu_reference
from helpers import make_inputs, rel_err

pytestmark = pytest.mark.gpu

TOL = 2e-2

# id, batch, n_q, n_k, heads, kv_heads, causal (C ABI code), head_dim
SHAPES = [
    # 18 key blocks x 32 (batch, head) pairs > 512 resident workgroups: mirror pairs
    ("mirror_pairs_even", 16, 2304, 2304, 2, 2, 1, 64),
    # 17 key blocks: the middle block has no mirror
    ("mirror_pairs_odd", 16, 2176, 2176, 2, 2, 1, 64),
    # grouped heads (4 query heads per key/value head) with mirror pairs
    ("mirror_pairs_gqa4", 8, 2304, 2304, 16, 4, 1, 64),
    # top-left causal, N_K > N_Q: key blocks past N_Q see no query (empty blocks in pairs)
    ("mirror_pairs_empty_blocks", 16, 1024, 2304, 2, 2, 1, 64),
    # bottom-right causal with N_Q > N_K
    ("mirror_pairs_bottom_right", 16, 2600, 2304, 2, 2, 2, 64),
    # D = 128 (64-key blocks, no mirror pairs): 32 blocks x 32 pairs, rank-major
    ("d128_rank_major", 16, 2048, 2048, 2, 2, 1, 128),
    # 33 blocks, the last one ragged
    ("d128_ragged_last_block", 16, 2100, 2100, 2, 2, 1, 128),
    # grouped heads, bottom-right causal with N_Q > N_K
    ("d128_gqa4_bottom_right", 4, 2600, 2304, 16, 4, 2, 128),
    # top-left causal, N_K > N_Q: key blocks no query sees
    ("d128_empty_blocks", 16, 1024, 2304, 2, 2, 1, 128),
    # 16 blocks x 288 pairs = 9 rounds of 512 workgroups: chunked grid order
    ("d128_chunked", 144, 1024, 1024, 2, 2, 1, 128),
    # D = 256 (the 32-key kernel at one wave per SIMD, 256 resident workgroups):
    # 18 key blocks x 32 pairs, mirror pairs without the skew
    ("d256_mirror_pairs", 16, 2304, 2304, 2, 2, 1, 256),
]


def _reference_residual(x, scale, causal, dtype):
    """O (fp32 forward, rounded to dtype) and L from gpu_reference, over all heads,
    for top-left (1) or bottom-right (2) masks."""
    B, Nq, H, _ = x["q"].shape
    Hk = x["k"].shape[2]
    G = H // Hk
    o = torch.empty_like(x["q"], dtype=torch.float32)
    lse = torch.empty((B, H, Nq), device=x["q"].device)
    for b in range(B):
        for h in range(H):
            q = x["q"][b, :, h].float()
            k = x["k"][b, :, h // G].float()
            v = x["v"][b, :, h // G].float()
            o[b, :, h], lse[b, h] = _fwd_head(q, k, v, scale, causal)
    return o.to(dtype), lse


def _mask(n_q, n_k, causal, device):
    off = n_k - n_q if causal == 2 else 0
    return torch.arange(n_k, device=device)[None, :] <= torch.arange(n_q, device=device)[:, None] + off


def _fwd_head(q, k, v, scale, causal):
    s = torch.mm(q, k.t().contiguous()) * scale
    s = s.masked_fill(~_mask(q.shape[0], k.shape[0], causal, q.device), float("-inf"))
    lse = torch.logsumexp(s, dim=-1)
    p = torch.exp(s - lse[:, None]).nan_to_num(0.0)  # rows without keys: P = 0
    return torch.mm(p, v), torch.where(torch.isinf(lse), torch.full_like(lse, float("inf")), lse)


def _bwdbwd_head(q, k, v, o, do, ddq, ddk, ddv, lse, scale, causal):
    """gpu_reference.bwdbwd_head with a general causal mask (top-left or bottom-right)."""
    mm = torch.mm
    s = mm(q, k.t().contiguous()) * scale
    s = s.masked_fill(~_mask(q.shape[0], k.shape[0], causal, q.device), float("-inf"))
    p = torch.exp(s - lse[:, None])
    dp = mm(do, v.t().contiguous())
    dds = scale * (mm(ddq, k.t().contiguous()) + mm(q, ddk.t().contiguous()))
    d = (o * do).sum(-1)
    dd = (dds * p).sum(-1)
    dp2 = mm(do, ddv.t().contiguous()) - dp * dd[:, None] - dds * d[:, None] + dp * dds
    b = (dp2 * p).sum(-1)
    ds = scale * p * (dp - d[:, None])
    ds2 = scale * p * (dp2 - b[:, None])
    ddp = p * (dds - dd[:, None])
    return mm(ds, ddk) + mm(ds2, k), mm(ds.t().contiguous(), ddq) + mm(ds2.t().contiguous(), q), \
        mm(ddp.t().contiguous(), do), mm(p, ddv) + mm(ddp, v)


@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_stage2_grid_layouts(shape, cuda_device):
    from flash_hog import _hip

    name, B, Nq, Nk, H, Hk, causal, D = shape
    print("[case] stage-2 grid", name, flush=True)
    dtype = torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=71, kv_heads=Hk, device=cuda_device)
    o, lse = _reference_residual(x, scale, causal, dtype)
    outs = _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"], lse, causal,
                                 scale)
    torch.cuda.synchronize()
    G = H // Hk
    ref = [torch.zeros_like(t, dtype=torch.float32) for t in outs]
    for b in range(B):
        for h in range(H):
            hk = h // G
            args = [x["q"][b, :, h], x["k"][b, :, hk], x["v"][b, :, hk], o[b, :, h], x["do"][b, :, h],
                    x["ddq"][b, :, h], x["ddk"][b, :, hk], x["ddv"][b, :, hk]]
            dq2, dk2, dv2, ddo = _bwdbwd_head(*(a.float() for a in args), lse[b, h], scale, causal)
            ref[0][b, :, h] = dq2
            ref[1][b, :, hk] += dk2
            ref[2][b, :, hk] += dv2
            ref[3][b, :, h] = ddo
    for label, a, r in zip(("dq2", "dk2", "dv2", "ddo"), outs, ref):
        assert torch.isfinite(a).all(), label
        err = rel_err(a, r)
        assert err < TOL, f"{name} {label}: rel err {err:.3e}"
    if causal == 1 and Nk > Nq:
        # keys past the last query see no query: their gradients are exactly zero
        assert not outs[1][:, Nq:].any() and not outs[2][:, Nq:].any()
