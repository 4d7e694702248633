"""The first backward on grids of several rounds of resident workgroups.

Both kernels of the first backward (dQ tiled over 128-query blocks, dK/dV over
128-key blocks) issue their causal blocks longest first, one block per
workgroup, with (batch, head) as the minor index (in chunks of pairs when the
grid is longer than 8 rounds). These shapes give grids of one to several
rounds, odd block counts, grouped heads, blocks that see nothing (top-left
causal with N_K > N_Q, bottom-right with N_Q > N_K), D = 128 and D = 256. Each shape is
checked on every (batch, head) against an fp32 closed form on the GPU (the
first backward of tests/gpu_reference.py with a general causal mask), with
the residual (O, L) from the fp32 forward. Tolerance: max|a - r| / max|r| <
2e-2 (bf16 against an fp32 reference).
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import make_inputs, rel_err
from test_gpu_stage2_grids import _mask, _reference_residual

pytestmark = pytest.mark.gpu

TOL = 2e-2

# id, batch, n_q, n_k, heads, kv_heads, causal (C ABI code), head_dim
SHAPES = [
    # 18 blocks x 32 (batch, head) pairs: a little over one round of 512 resident workgroups
    ("rounds_1.1", 16, 2304, 2304, 2, 2, 1, 64),
    # 16 blocks x 64 pairs: two rounds (the standard configuration's grid)
    ("rounds_2", 32, 2048, 2048, 2, 2, 1, 64),
    # 17 blocks, the last one ragged
    ("odd_blocks", 16, 2176, 2176, 2, 2, 1, 64),
    # grouped heads (4 query heads per key/value head)
    ("gqa4", 8, 2304, 2304, 16, 4, 1, 64),
    # top-left causal, N_K > N_Q: key blocks past N_Q see no query
    ("empty_key_blocks", 16, 1024, 2304, 2, 2, 1, 64),
    # bottom-right causal with N_Q > N_K: leading query rows see no key
    ("bottom_right", 16, 2600, 2304, 2, 2, 2, 64),
    # D = 128 (one wave per SIMD, 256 resident workgroups): two rounds
    ("d128", 16, 2048, 2048, 2, 2, 1, 128),
    # D = 256: the dK/dV kernel runs twice, for the two halves of the output columns
    ("d256_gqa2", 4, 1100, 1100, 4, 2, 1, 256),
]


def _bwd_head(q, k, v, o, do, lse, scale, causal):
    s = torch.mm(q, k.t().contiguous()) * scale
    s = s.masked_fill(~_mask(q.shape[0], k.shape[0], causal, q.device), float("-inf"))
    p = torch.exp(s - lse[:, None])  # rows without keys: L = +inf, P = 0
    d = (o * do).sum(-1)
    ds = scale * p * (torch.mm(do, v.t().contiguous()) - d[:, None])
    return torch.mm(ds, k), torch.mm(ds.t().contiguous(), q), torch.mm(p.t().contiguous(), do), d


@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_bwd_grid_layouts(shape, cuda_device):
    from flash_hog import _hip

    name, B, Nq, Nk, H, Hk, causal, D = shape
    print("[case] first-backward grid", name, flush=True)
    dtype = torch.bfloat16
    scale = 1.0 / math.sqrt(D)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=73, kv_heads=Hk, device=cuda_device)
    o, lse = _reference_residual(x, scale, causal, dtype)
    outs = _hip.attention_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, causal, scale)
    torch.cuda.synchronize()
    G = H // Hk
    ref = [torch.zeros_like(t, dtype=torch.float32) for t in outs]
    for b in range(B):
        for h in range(H):
            hk = h // G
            args = [x["q"][b, :, h], x["k"][b, :, hk], x["v"][b, :, hk], o[b, :, h], x["do"][b, :, h]]
            dq, dk, dv, d = _bwd_head(*(a.float() for a in args), lse[b, h], scale, causal)
            ref[0][b, :, h] = dq
            ref[1][b, :, hk] += dk
            ref[2][b, :, hk] += dv
            ref[3][b, h] = d
    for label, a, r in zip(("dq", "dk", "dv", "D"), outs, ref):
        assert torch.isfinite(a).all(), label
        err = rel_err(a, r)
        assert err < TOL, f"{name} {label}: rel err {err:.3e}"
    if causal == 1 and Nk > Nq:
        # keys past the last query see no query: their gradients are exactly zero
        assert not outs[1][:, Nq:].any() and not outs[2][:, Nq:].any()
