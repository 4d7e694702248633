"""The first backward's alternative kernels for 2-byte types at D = 64.

The dK/dV work runs in the kernel with 64 keys per wave and a generated sweep
(fhog_bwd_k64.hip) or in the compiled one (bwd_k_kernel in fhog_bwd.hip, 32
keys per wave at two waves per SIMD), the dQ work in the kernel with 64
queries per wave and a generated sweep (fhog_bwd_q64.hip) or in the compiled
bwd_q_kernel: by default the one-wave kernel when its grid fills whole rounds
of resident workgroups, else the compiled one; FLASH_HOG_BWD = k64 or
compiled and FLASH_HOG_BWDQ = q64 or compiled force either kernel.

The other suites run the defaults. Here every D = 64 bf16 and fp16 case of
the parity, scale and random-sweep suites and every D = 64 shape of the
first-backward grid suite runs again with each alternative selected, against
the fp64 oracle (or the fp32 closed form on the GPU) at the same tolerances,
and full-size shapes compare each pair of kernels on the same inputs
(grouped heads, a ragged fp16 shape, bottom-right causal). The generated
sweeps' control flow and hazard distances are checked on the CPU
(tests/test_bwd_k64_loop_control.py, tests/test_bwd_q64_loop_control.py).
"""

from __future__ import annotations

import pytest
import torch

import test_gpu_bwd_grids as grids
import test_gpu_parity as parity
import test_gpu_sweep as sweep
from helpers import default_scale, make_inputs

pytestmark = pytest.mark.gpu


VARIANTS = {"dkdv_compiled": ("FLASH_HOG_BWD", "compiled"), "dkdv_k64": ("FLASH_HOG_BWD", "k64"),
            "dq_q64": ("FLASH_HOG_BWDQ", "q64"), "dq_compiled": ("FLASH_HOG_BWDQ", "compiled")}


@pytest.fixture(params=sorted(VARIANTS))
def variant(request, monkeypatch):
    monkeypatch.setenv(*VARIANTS[request.param])
    return request.param


def _two_byte_d64(cases, dim, dtype):
    return [c for c in cases if c[dim] == 64 and c[dtype] in (torch.bfloat16, torch.float16)]


CASES = _two_byte_d64(parity.CASES, 6, 7)
SCALE_CASES = _two_byte_d64(parity.SCALE_CASES, 6, 7)
PROBLEMS = _two_byte_d64(sweep.PROBLEMS, 6, 7)
SHAPES = [s for s in grids.SHAPES if s[7] == 64]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_variant_bwd_matches_oracle(case, cuda_device, variant):
    parity.test_bwd_matches_oracle(case, cuda_device)


@pytest.mark.parametrize("case", SCALE_CASES, ids=[c[0] for c in SCALE_CASES])
def test_variant_other_scales(case, cuda_device, variant):
    parity.test_all_kernels_other_scales(case, cuda_device)


@pytest.mark.parametrize("problem", PROBLEMS, ids=[p[0] for p in PROBLEMS])
def test_variant_random_problem(problem, cuda_device, variant):
    sweep.test_random_problem_all_kernels(problem, cuda_device)


@pytest.mark.parametrize("shape", SHAPES, ids=[s[0] for s in SHAPES])
def test_variant_grid_layouts(shape, cuda_device, variant):
    grids.test_bwd_grid_layouts(shape, cuda_device)


# (id, batch, n, heads, kv_heads, causal, dtype)
FULL = [("b4_n2048_h16_causal", 4, 2048, 16, 16, 1, torch.bfloat16),
        ("b2_n1000_h8_gqa4_noncausal", 2, 1000, 8, 2, 0, torch.bfloat16),
        ("b8_n1000_h12_noncausal_fp16", 8, 1000, 12, 12, 0, torch.float16),
        ("b1_n4000_h4_bottom_right", 1, 4000, 4, 4, 2, torch.bfloat16)]


@pytest.mark.parametrize("case", FULL, ids=[c[0] for c in FULL])
def test_k64_matches_compiled_full_size(case, cuda_device, monkeypatch):
    """Both dK/dV kernels on the same inputs give the same bits: they form the
    same products in the same order (the one-wave kernel's constants operand
    holds the fp32 start values exactly, in three bf16 parts), which is what
    lets launch_bwd choose between them by grid shape without a result
    depending on the batch a problem is part of."""
    name, B, N, H, Hk, causal, dtype = case
    print(f"[case] k64 vs compiled {name}", flush=True)
    from flash_hog import _hip

    x = make_inputs(B, N, N, H, 64, dtype, seed=9, kv_heads=Hk)
    g = lambda t: t.to(cuda_device)
    scale = default_scale(64)
    o, lse = _hip.attention_fwd(g(x["q"]), g(x["k"]), g(x["v"]), causal, scale)
    args = (g(x["q"]), g(x["k"]), g(x["v"]), o, g(x["do"]), lse, causal, scale)
    outs = {}
    for which in ("compiled", "k64"):  # any other value than "compiled" selects k64
        monkeypatch.setenv("FLASH_HOG_BWD", which)
        outs[which] = _hip.attention_bwd(*args)
        torch.cuda.synchronize()
    for a, b, label in zip(outs["k64"], outs["compiled"], ("dq", "dk", "dv", "D")):
        assert torch.isfinite(a).all(), label
        print(f"  {label}: max abs diff {(a.float() - b.float()).abs().max().item():.3e}", flush=True)
        assert torch.equal(a, b), f"{label}: k64 and compiled differ"


@pytest.mark.parametrize("case", FULL, ids=[c[0] for c in FULL])
def test_q64_matches_compiled_full_size(case, cuda_device, monkeypatch):
    """Both dQ kernels on the same inputs give the same bits (the same products
    in the same order, D summed by the same dot8)."""
    name, B, N, H, Hk, causal, dtype = case
    print(f"[case] q64 vs compiled {name}", flush=True)
    from flash_hog import _hip

    x = make_inputs(B, N, N, H, 64, dtype, seed=9, kv_heads=Hk)
    g = lambda t: t.to(cuda_device)
    scale = default_scale(64)
    o, lse = _hip.attention_fwd(g(x["q"]), g(x["k"]), g(x["v"]), causal, scale)
    args = (g(x["q"]), g(x["k"]), g(x["v"]), o, g(x["do"]), lse, causal, scale)
    outs = {}
    for which in ("compiled", "q64"):
        monkeypatch.setenv("FLASH_HOG_BWDQ", which)
        outs[which] = _hip.attention_bwd(*args)
        torch.cuda.synchronize()
    for a, b, label in zip(outs["q64"], outs["compiled"], ("dq", "dk", "dv", "D")):
        assert torch.isfinite(a).all(), label
        print(f"  {label}: max abs diff {(a.float() - b.float()).abs().max().item():.3e}", flush=True)
        assert torch.equal(a, b), f"{label}: q64 and compiled differ"
