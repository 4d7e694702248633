"""A seeded sweep of small random problems through every kernel, against the
fp64 oracle.

The hand-picked cases of test_gpu_parity.py cover each feature on its own;
this sweep mixes them: batch 1-3, query and key lengths 1-300 drawn
independently (ragged tails, N_Q != N_K, single tokens), 1-8 query heads with
a random divisor as key/value heads (MHA, GQA, MQA), head dim 64, 128 or 256
(64 or 128 in fp32), bf16 / fp16 / fp32, no mask / top-left / bottom-right
causal (rows without
keys included), and the default or a random softmax scale, negative ones
included. Each problem runs the forward, the first backward and the double
backward through the C ABI; O, L, dQ, dK, dV, D, dQ2, dK2, dV2, ddO and the row
statistics D, dD, B are compared with oracle/attention.py on the same inputs.
Tolerances are those of tests/helpers.py (max|a - r| / max|r| < 1e-3 for fp32,
< 2e-2 for the 2-byte types).
"""

from __future__ import annotations

import random

import pytest
import torch

from helpers import DEGENERATE_FLOOR, TOL, make_inputs, rel_err, stat_errs, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32


def _problems(count=36, seed=2024):
    rnd = random.Random(seed)
    out = []
    for i in range(count):
        dtype = rnd.choice((BF16, BF16, F16, F32))
        D = rnd.choice((64, 128) if dtype == F32 else (64, 128, 256))
        H = rnd.choice((1, 2, 3, 4, 6, 8))
        Hk = rnd.choice([d for d in range(1, H + 1) if H % d == 0])
        B = rnd.choice((1, 2, 3))
        nq = rnd.choice((1, rnd.randint(2, 300), rnd.randint(2, 300)))
        nk = rnd.choice((nq, rnd.randint(1, 300)))
        causal = rnd.choice((0, 1, 2))
        scale = rnd.choice((None, round(rnd.uniform(0.05, 0.2), 4), -round(rnd.uniform(0.05, 0.2), 4)))
        out.append((f"p{i:02d}", B, nq, nk, H, Hk, D, dtype, causal, scale))
    return out


PROBLEMS = _problems()

# Two problems of a larger run of the same generator (250 problems, seed 7) whose ddO and dQ2 exceeded the
# bf16 tolerance (2.000e-2 and 2.07e-2) before the fused stage 1 subtracted dD O with dD summed over the
# bf16-rounded P ddS its ddO products take: rows that see few keys (N_K = 34 under a top-left mask), and
# D = 256 with scale 0.199. A CPU model of the kernel's roundings puts them at 0.009 and 0.010 now.
PROBLEMS += [("p44", 2, 266, 239, 2, 2, 256, BF16, 0, 0.199), ("p74", 2, 298, 34, 2, 1, 64, BF16, 1, None)]
# A problem of a 250-problem run with seed 31 (its p07, inputs seeded with 108): one query row whose B is
# the small difference of c = D dD + B = 0.284 and D dD = 0.269. The fused stage 1's B is then 17 % off
# relative to B itself but 0.9 % of c, the scale at which pass 4 uses it (tests/helpers.py b_stat_err,
# tests/test_rounding_model.py). All four outputs are within tolerance.
PROBLEMS += [("s31p07", 1, 1, 78, 1, 1, 128, BF16, 0, 0.1247, 108)]
# A problem of a 250-problem run with seed 79 (its p08, inputs seeded with 109): four queries, D = 256,
# bottom-right mask. B formed as <dO, ddO> - D dD put dK2 at 2.21e-2 against the 2e-2 bar; with B summed
# from unrounded per-pair terms it is within tolerance (tests/test_rounding_model.py).
PROBLEMS += [("s79p08", 1, 4, 201, 3, 3, 256, BF16, 2, 0.1843, 109)]


def _lse_err(lse, lse_ref):
    got, ref = to_np(lse), lse_ref
    import numpy as np

    empty = np.isposinf(ref)
    assert np.array_equal(np.isposinf(got), empty), "rows without keys must have L = +inf"
    if empty.all():
        return 0.0
    return float(np.max(np.abs(got[~empty] - ref[~empty])) / max(1.0, np.max(np.abs(ref[~empty]))))


@pytest.mark.parametrize("problem", PROBLEMS, ids=[p[0] for p in PROBLEMS])
def test_random_problem_all_kernels(problem, cuda_device):
    from flash_hog import _hip

    name, B, Nq, Nk, H, Hk, D, dtype, causal, scale = problem[:10]
    seed = problem[10] if len(problem) > 10 else 101 + int(name[1:])
    scale = D ** -0.5 if scale is None else scale
    print(f"[case] sweep {name}: B{B} Nq{Nq} Nk{Nk} H{H}/{Hk} D{D} {dtype} causal={causal} scale={scale}",
          flush=True)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=seed, kv_heads=Hk)
    g = lambda t: t.to(cuda_device)
    tol = TOL[dtype]

    o, lse = _hip.attention_fwd(g(x["q"]), g(x["k"]), g(x["v"]), causal, scale)
    torch.cuda.synchronize()
    o_ref, lse_ref = ora.attn_fwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), scale, causal)
    assert rel_err(o, o_ref, DEGENERATE_FLOOR) < tol, "O"
    assert _lse_err(lse, lse_ref) < 1e-3, "L"

    # The backward passes take the oracle's residual, so that each kernel is
    # checked on its own.
    o32 = torch.from_numpy(o_ref).to(dtype)
    l32 = torch.from_numpy(lse_ref).float()
    dq, dk, dv, delta = _hip.attention_bwd(g(x["q"]), g(x["k"]), g(x["v"]), g(o32), g(x["do"]), g(l32), causal,
                                           scale)
    torch.cuda.synchronize()
    ref = ora.attn_bwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), to_np(o32), to_np(x["do"]), to_np(l32),
                       scale, causal)
    for a, r, label in zip((dq, dk, dv, delta), ref, ("dq", "dk", "dv", "D")):
        err = rel_err(a, r, DEGENERATE_FLOOR)
        assert err < tol, f"{label}: rel err {err:.3e}"

    dq2, dk2, dv2, ddo, stats = _hip.attention_bwdbwd(
        g(x["q"]), g(x["k"]), g(x["v"]), g(o32), g(x["do"]), g(x["ddq"]), g(x["ddk"]), g(x["ddv"]), g(l32),
        causal, scale, return_stats=True)
    torch.cuda.synchronize()
    ref = ora.attn_bwd_bwd_stats(*(to_np(x[n]) for n in ("q", "k", "v")), to_np(o32), to_np(x["do"]),
                                 *(to_np(x[n]) for n in ("ddq", "ddk", "ddv")), to_np(l32), scale, causal,
                                 return_stats=True)
    for a, r, label in zip((dq2, dk2, dv2, ddo), ref[:4], ("dq2", "dk2", "dv2", "ddo")):
        err = rel_err(a, r, DEGENERATE_FLOOR)
        assert err < tol, f"{label}: rel err {err:.3e}"
    for err, label in zip(stat_errs(tuple(stats), ref[4:]), ("D", "dD", "B")):
        assert err < tol, f"{label}: rel err {err:.3e}"
