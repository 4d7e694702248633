"""The forward's lazy rescale on logits whose row maximum jumps late.

The forward forms each tile's probabilities with the row's running maximum
(possibly stale) and takes the exact maximum, rescaling O and l, only when a
lane's 16 probabilities sum to more than 2^8 or overflow. With N(0, 1) inputs
that happens on a row's first tile and rarely after. Here the last 64 keys are
multiplied by 6 (maxima jump by tens of log2 units, many slow-path tiles) or by
100 (the stale-maximum exponent reaches the hundreds, so P overflows to inf
before the rescale), across dtypes, head dims and masks. O and L are compared
with the fp64 oracle forward (oracle/attention.py attn_fwd) under the parity
tolerances of tests/helpers.py; L to 1e-3 of max(1, max|L|).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import DEGENERATE_FLOOR, TOL, default_scale, make_inputs, rel_err, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

F32, F16, BF16 = torch.float32, torch.float16, torch.bfloat16
NONE, TL, BR = 0, 1, 2

# (id, batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, tail factor)
CASES = [
    ("bf16_causal_tail_x6", 1, 512, 512, 2, 2, 64, BF16, TL, 6.0),
    ("bf16_noncausal_tail_x100", 1, 300, 300, 2, 1, 64, BF16, NONE, 100.0),
    ("f16_d128_bottom_right_tail_x6", 1, 200, 333, 2, 2, 128, F16, BR, 6.0),
    ("f32_causal_tail_x100", 1, 256, 256, 2, 2, 64, F32, TL, 100.0),
    ("bf16_d256_noncausal_tail_x6", 1, 160, 160, 2, 2, 256, BF16, NONE, 6.0),
]


def _lse_err(got, ref):
    got = got.detach().cpu().double().numpy()
    empty = np.isinf(ref)
    if empty.any():
        assert np.all(np.isinf(got[empty]) & (got[empty] > 0))
    return float(np.max(np.abs(got[~empty] - ref[~empty])) / max(1.0, np.max(np.abs(ref[~empty]))))


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fwd_late_jumps_match_oracle(case, cuda_device):
    from flash_hog import _hip

    name, B, Nq, Nk, H, Hk, D, dtype, causal, tail = case
    print("[case] fwd sharp", name, flush=True)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=5, kv_heads=Hk)
    k = x["k"].float()
    k[:, Nk - 64:] *= tail
    k = k.to(dtype)
    scale = default_scale(D)
    o, lse = _hip.attention_fwd(x["q"].to(cuda_device), k.to(cuda_device), x["v"].to(cuda_device), causal, scale)
    torch.cuda.synchronize()
    o_ref, lse_ref = ora.attn_fwd(to_np(x["q"]), to_np(k), to_np(x["v"]), scale, causal)
    assert np.isfinite(lse_ref[~np.isinf(lse_ref)]).all()
    assert torch.isfinite(o).all(), name
    err = rel_err(o, o_ref, DEGENERATE_FLOOR)
    assert err < TOL[dtype], f"{name}: O rel err {err:.3e}"
    assert _lse_err(lse, lse_ref) < 1e-3, name
