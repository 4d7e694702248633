"""The second stage-2 kernel for bf16 at D = 64 (fhog_bwdbwd_k32.hip: 32 keys
per wave at one wave per SIMD, generated sweep), which FLASH_HOG_STAGE2=k32
selects at launch.

Every D = 64 bf16 case of the parity, scale, single-key and random-sweep
suites runs again with it selected, against the fp64 oracle and at the same
tolerances (rows that see no key included: their L = +inf must not reach the
per-query constants operand); the standard full-size configuration compares
its dK2 and dV2 with the compiled kernel's on the same inputs. Its control
flow and hazard distances are checked on the CPU
(tests/test_k32_loop_control.py).
"""

from __future__ import annotations

import pytest
import torch

import test_gpu_parity as parity
import test_gpu_sweep as sweep
from helpers import DEGENERATE_FLOOR, default_scale, make_inputs, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture
def k32(monkeypatch):
    monkeypatch.setenv("FLASH_HOG_STAGE2", "k32")


def _bf16_d64(cases, dim, dtype):
    return [c for c in cases if c[dim] == 64 and c[dtype] == torch.bfloat16]


CASES = _bf16_d64(parity.CASES, 6, 7)
SCALE_CASES = _bf16_d64(parity.SCALE_CASES, 6, 7)
SINGLE_KEY_CASES = _bf16_d64(parity.SINGLE_KEY_CASES, 6, 7)
PROBLEMS = _bf16_d64(sweep.PROBLEMS, 6, 7)


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_k32_bwdbwd_matches_oracle(case, cuda_device, k32):
    parity.test_bwdbwd_matches_oracle(case, cuda_device)


@pytest.mark.parametrize("case", SCALE_CASES, ids=[c[0] for c in SCALE_CASES])
def test_k32_other_scales(case, cuda_device, k32):
    parity.test_all_kernels_other_scales(case, cuda_device)


@pytest.mark.parametrize("case", SINGLE_KEY_CASES, ids=[c[0] for c in SINGLE_KEY_CASES])
def test_k32_single_key_rows_are_exact(case, cuda_device, k32):
    parity.test_single_key_rows_are_exact(case, cuda_device)


@pytest.mark.parametrize("problem", PROBLEMS, ids=[p[0] for p in PROBLEMS])
def test_k32_random_problem(problem, cuda_device, k32):
    sweep.test_random_problem_all_kernels(problem, cuda_device)


# (id, batch, n, heads, kv_heads, causal)
FULL = [("b4_n2048_h16_causal", 4, 2048, 16, 16, 1), ("b2_n1000_h8_gqa4_noncausal", 2, 1000, 8, 2, 0)]


@pytest.mark.parametrize("case", FULL, ids=[c[0] for c in FULL])
def test_k32_matches_compiled_full_size(case, cuda_device, monkeypatch):
    """Both stage-2 kernels on the same inputs: dK2 and dV2 agree to a few
    bf16 ulps (different summation orders of the same fp32 terms)."""
    name, B, N, H, Hk, causal = case
    print(f"[case] k32 vs compiled {name}", flush=True)
    from flash_hog import _hip

    x = make_inputs(B, N, N, H, 64, torch.bfloat16, seed=9, kv_heads=Hk)
    g = lambda t: t.to(cuda_device)
    scale = default_scale(64)
    o, lse = _hip.attention_fwd(g(x["q"]), g(x["k"]), g(x["v"]), causal, scale)
    args = (g(x["q"]), g(x["k"]), g(x["v"]), o, g(x["do"]), g(x["ddq"]), g(x["ddk"]), g(x["ddv"]), lse, causal,
            scale)
    outs = {}
    for which in ("compiled", "k32"):
        monkeypatch.setenv("FLASH_HOG_STAGE2", which)
        dq2, dk2, dv2, ddo = _hip.attention_bwdbwd(*args)
        torch.cuda.synchronize()
        outs[which] = (dk2, dv2)
    for a, b, label in zip(outs["k32"], outs["compiled"], ("dk2", "dv2")):
        err = rel_err(a, b.float().cpu().numpy(), DEGENERATE_FLOOR)
        print(f"  {label}: {err:.2e}", flush=True)
        assert err < 1e-2, f"{label}: k32 vs compiled rel err {err:.3e}"
