"""The fused stage-1 kernel at D = 64 for 2-byte types
(fhog_bwdbwd_fused.hip: 16 queries per wave, two waves per SIMD), which
FLASH_HOG_STAGE1=fused selects at launch in place of the default 32-query
kernel (fhog_bwdbwd_q32.hip) that every other D = 64 test runs.

Every D = 64 2-byte case of the parity, scale, single-key and random-sweep
suites runs again with it selected, against the fp64 oracle and at the same
tolerances; the standard and ragged full-size configurations compare the two
kernels' outputs on the same inputs. The q32 kernel's control flow and hazard
distances are checked on the CPU (tests/test_q32_loop_control.py).
"""

from __future__ import annotations

import pytest
import torch

import test_gpu_parity as parity
import test_gpu_sweep as sweep
from helpers import DEGENERATE_FLOOR, default_scale, make_inputs, rel_err

pytestmark = pytest.mark.gpu

TWO_BYTE = (torch.bfloat16, torch.float16)


@pytest.fixture
def fused(monkeypatch):
    monkeypatch.setenv("FLASH_HOG_STAGE1", "fused")


def _d64(cases, dim, dtype):
    return [c for c in cases if c[dim] == 64 and c[dtype] in TWO_BYTE]


CASES = _d64(parity.CASES, 6, 7)
SCALE_CASES = _d64(parity.SCALE_CASES, 6, 7)
SINGLE_KEY_CASES = _d64(parity.SINGLE_KEY_CASES, 6, 7)
PROBLEMS = _d64(sweep.PROBLEMS, 6, 7)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_fused_d64_bwdbwd_matches_oracle(case, cuda_device, fused):
    parity.test_bwdbwd_matches_oracle(case, cuda_device)


@pytest.mark.parametrize("case", SCALE_CASES, ids=[c[0] for c in SCALE_CASES])
def test_fused_d64_other_scales(case, cuda_device, fused):
    parity.test_all_kernels_other_scales(case, cuda_device)


@pytest.mark.parametrize("case", SINGLE_KEY_CASES, ids=[c[0] for c in SINGLE_KEY_CASES])
def test_fused_d64_single_key_rows_are_exact(case, cuda_device, fused):
    parity.test_single_key_rows_are_exact(case, cuda_device)


@pytest.mark.parametrize("problem", PROBLEMS, ids=[p[0] for p in PROBLEMS])
def test_fused_d64_random_problem(problem, cuda_device, fused):
    sweep.test_random_problem_all_kernels(problem, cuda_device)


# (id, batch, n, heads, dtype, causal)
FULL = [("b4_n2048_h16_bf16_causal", 4, 2048, 16, torch.bfloat16, 1),
        ("b8_n1000_h12_f16_noncausal", 8, 1000, 12, torch.float16, 0)]


@pytest.mark.parametrize("case", FULL, ids=[c[0] for c in FULL])
def test_q32_matches_fused_full_size(case, cuda_device, monkeypatch):
    """Both stage-1 kernels on the same full-size inputs: dQ2, ddO and the row
    statistics agree to a few bf16 ulps (the kernels sum in different orders
    and round the same fp32 values)."""
    name, B, N, H, dtype, causal = case
    print(f"[case] q32 vs fused {name}", flush=True)
    from flash_hog import _hip

    x = make_inputs(B, N, N, H, 64, dtype, seed=5)
    g = lambda t: t.to(cuda_device)
    scale = default_scale(64)
    o, lse = _hip.attention_fwd(g(x["q"]), g(x["k"]), g(x["v"]), causal, scale)
    args = (g(x["q"]), g(x["k"]), g(x["v"]), o, g(x["do"]), g(x["ddq"]), g(x["ddk"]), g(x["ddv"]), lse, causal,
            scale)
    outs = {}
    for which in ("fused", "q32"):
        monkeypatch.setenv("FLASH_HOG_STAGE1", which)
        dq2, dk2, dv2, ddo, stats = _hip.attention_bwdbwd(*args, return_stats=True)
        torch.cuda.synchronize()
        outs[which] = (dq2, dk2, dv2, ddo) + tuple(stats)
    for a, b, label in zip(outs["q32"], outs["fused"], ("dq2", "dk2", "dv2", "ddo", "D", "dD", "B")):
        err = rel_err(a, b.float().cpu().numpy(), DEGENERATE_FLOOR)
        print(f"  {label}: {err:.2e}", flush=True)
        assert err < 1e-2, f"{label}: q32 vs fused rel err {err:.3e}"
