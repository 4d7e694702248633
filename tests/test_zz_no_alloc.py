"""fhog_attention_bwdbwd_noalloc against fhog_attention_bwdbwd.

The allocation-free entry point keeps the row statistics D, dD, B in the
library's static device scratch instead of a caller-owned workspace and runs
the same kernels, so its outputs must equal the workspace entry point's bit
for bit. Two calls in a row, the second on a smaller problem, check that the
scratch left by one call does not leak into the next; a third call reuses the
first call's output buffers.
"""

from __future__ import annotations

import math

import pytest
import torch

from helpers import make_inputs

pytestmark = pytest.mark.gpu

BF16, F16 = torch.bfloat16, torch.float16

# batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal (C ABI code), seed
CALLS = [
    (2, 1024, 1024, 8, 8, 64, BF16, 1, 61),
    (1, 300, 300, 4, 2, 64, BF16, 1, 62),
    (1, 200, 260, 2, 2, 128, F16, 2, 63),
]


def _run(case, device):
    from flash_hog import _hip

    B, Nq, Nk, H, Hk, D, dtype, causal, seed = case
    print("[case] noalloc", case, flush=True)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=seed, kv_heads=Hk, device=device)
    scale = 1.0 / math.sqrt(D)
    o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
    args = (x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"], lse, causal, scale)
    ref = _hip.attention_bwdbwd(*args)
    got = _hip.attention_bwdbwd_noalloc(*args)
    torch.cuda.synchronize()
    return args, ref, got


def test_noalloc_equals_workspace_entry_point(cuda_device):
    from flash_hog import _hip

    first = None
    for case in CALLS:
        args, ref, got = _run(case, cuda_device)
        for name, a, r in zip(("dq2", "dk2", "dv2", "ddo"), got, ref):
            assert torch.equal(a, r), f"{case}: {name} differs from fhog_attention_bwdbwd"
        if first is None:
            first = (args, ref, got)
    # the first problem again, into its own (already written) output buffers
    args, ref, got = first
    for t in got:
        t.fill_(float("nan"))
    again = _hip.attention_bwdbwd_noalloc(*args, out=got)
    torch.cuda.synchronize()
    for name, a, r in zip(("dq2", "dk2", "dv2", "ddo"), again, ref):
        assert torch.equal(a, r), f"repeat: {name} differs"
