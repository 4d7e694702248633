"""The double backward at the full sizes of the benchmark configurations.

Each configuration runs through the C ABI at its real shape. Parity is checked
against tests/gpu_reference.py (the closed form in fp32 on the GPU, one
(batch, head) at a time, on the same dtype-rounded inputs; it is pinned to the
fp64 oracle in test_gpu_parity.py), on every head where that is cheap and on a
fixed subset of heads otherwise, and through properties that hold at any size:

- every row of dS, dS2 and ddP sums to zero, so the key-sums of dK2 and dV2
  vanish (per batch, head and column);
- the double backward is linear in the cotangents (ddQ, ddK, ddV), so doubling
  them doubles every output (a power-of-two scale is exact in floating point;
  only values that cross the subnormal range may round differently);
- causally, rows [0, M) of dQ2 and ddO depend only on the first M keys, so a
  length-N run and a length-M run agree on them bit for bit;
- the extra device memory of a call (outputs plus three fp32 row vectors) grows
  linearly in N; no (N, N) buffer is allocated.

Tolerance: max|a - r| / max|r| < 2e-2 for bf16 and fp16 inputs (the parity bar
for 2-byte runs against an fp32 reference).
"""

from __future__ import annotations

import math

import pytest
import torch

import gpu_reference
from helpers import make_inputs, rel_err

pytestmark = pytest.mark.gpu

TOL_2BYTE = 2e-2


def _announce(*what):
    print("[case]", *what, flush=True)


def _setup(B, N, H, D, dtype, causal, qkv_scale, device, seed):
    from flash_hog import _hip

    x = make_inputs(B, N, N, H, D, dtype, seed=seed, qkv_scale=qkv_scale, device=device)
    scale = 1.0 / math.sqrt(D)
    o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
    return x, o, lse, scale


def _bwdbwd(x, o, lse, causal, scale, mul=1.0):
    from flash_hog import _hip

    return _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o, x["do"], x["ddq"] * mul, x["ddk"] * mul,
                                 x["ddv"] * mul, lse, causal, scale)


def _check_heads(x, o, lse, outs, scale, causal, heads):
    """gpu_reference on the listed (batch, head) pairs, against the kernel's outputs."""
    names = ("dq2", "dk2", "dv2", "ddo")
    worst = {n: 0.0 for n in names}
    for b, h in heads:
        sl = lambda t: t[b:b + 1, :, h:h + 1, :]
        ref = gpu_reference.bwdbwd(*(sl(x[n]) for n in ("q", "k", "v")), sl(o), sl(x["do"]),
                                   *(sl(x[n]) for n in ("ddq", "ddk", "ddv")), lse[b:b + 1, h:h + 1], scale,
                                   causal)
        for n, a, r in zip(names, outs, ref):
            worst[n] = max(worst[n], rel_err(sl(a), r))
    for n in names:
        assert worst[n] < TOL_2BYTE, f"{n}: rel err {worst[n]:.3e}"
    return worst


def _check_key_sums(outs, tol=TOL_2BYTE):
    """sum over keys of dK2 and dV2 is zero; measured against the summed magnitude."""
    for label, t in (("dk2", outs[1]), ("dv2", outs[2])):
        t = t.float()
        s = t.sum(dim=1).abs().max().item()
        mag = t.abs().sum(dim=1).max().item()
        assert s <= tol * mag, f"{label}: |sum over keys| {s:.3e} vs magnitude {mag:.3e}"


def test_standard_b4_n2048_h16_d64_bf16_causal(cuda_device):
    _announce("config standard B4 N2048 H16 D64 bf16 causal")
    B, N, H, D = 4, 2048, 16, 64
    x, o, lse, scale = _setup(B, N, H, D, torch.bfloat16, True, 1.0, cuda_device, seed=101)
    outs = _bwdbwd(x, o, lse, True, scale)
    torch.cuda.synchronize()
    _check_heads(x, o, lse, outs, scale, True, [(b, h) for b in range(B) for h in range(H)])
    _check_key_sums(outs)
    doubled = _bwdbwd(x, o, lse, True, scale, mul=2.0)
    for a, a2 in zip(outs, doubled):
        assert rel_err(a2, a.float() * 2) < 1e-6


def test_long_b2_n8192_h16_d128_bf16_causal(cuda_device):
    _announce("config long B2 N8192 H16 D128 bf16 causal")
    B, N, H, D = 2, 8192, 16, 128
    x, o, lse, scale = _setup(B, N, H, D, torch.bfloat16, True, 1.0, cuda_device, seed=202)
    outs = _bwdbwd(x, o, lse, True, scale)
    torch.cuda.synchronize()
    _check_heads(x, o, lse, outs, scale, True, [(0, 0), (0, 7), (1, 3), (1, 15)])
    _check_key_sums(outs)


def test_ragged_b8_n1000_h12_d64_f16_noncausal(cuda_device):
    _announce("config ragged B8 N1000 H12 D64 fp16 non-causal")
    B, N, H, D = 8, 1000, 12, 64
    x, o, lse, scale = _setup(B, N, H, D, torch.float16, False, 0.5, cuda_device, seed=303)
    outs = _bwdbwd(x, o, lse, False, scale)
    torch.cuda.synchronize()
    _check_heads(x, o, lse, outs, scale, False, [(b, h) for b in range(B) for h in range(H)])
    _check_key_sums(outs)


def test_very_long_b1_n32768_h8_d64_bf16_causal(cuda_device):
    """The full 32768-token run, checked on a 4096-token slice: its first 4096
    rows of dQ2 and ddO equal those of a 4096-token run bit for bit, and the
    4096-token run (all four outputs) matches gpu_reference."""
    _announce("config very long B1 N32768 H8 D64 bf16 causal")
    B, N, H, D, M = 1, 32768, 8, 64, 4096
    x, o, lse, scale = _setup(B, N, H, D, torch.bfloat16, True, 1.0, cuda_device, seed=404)
    outs = _bwdbwd(x, o, lse, True, scale)
    torch.cuda.synchronize()
    assert all(torch.isfinite(t).all() for t in outs)
    _check_key_sums(outs)

    xs = {n: t[:, :M].contiguous() for n, t in x.items()}
    os_, ls_ = o[:, :M].contiguous(), lse[:, :, :M].contiguous()
    short = _bwdbwd(xs, os_, ls_, True, scale)
    torch.cuda.synchronize()
    assert torch.equal(outs[0][:, :M], short[0]), "dq2 prefix"
    assert torch.equal(outs[3][:, :M], short[3]), "ddo prefix"
    _check_heads(xs, os_, ls_, short, scale, True, [(0, h) for h in range(H)])


def test_peak_memory_is_linear_in_n(cuda_device):
    """Extra device memory of one call (B1 H8 D64 bf16 causal) from N = 4096
    to 32768: the four outputs and the three fp32 row vectors, linear in N."""
    from flash_hog import _hip

    B, H, D = 1, 8, 64
    per_token = None
    for N in (4096, 8192, 16384, 32768):
        _announce("peak memory N", N)
        x, o, lse, scale = _setup(B, N, H, D, torch.bfloat16, True, 1.0, cuda_device, seed=7)
        torch.cuda.synchronize()
        torch.cuda.reset_peak_memory_stats(cuda_device)
        base = torch.cuda.memory_allocated(cuda_device)
        outs = _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"], lse,
                                     True, scale)
        torch.cuda.synchronize()
        extra = torch.cuda.max_memory_allocated(cuda_device) - base
        exact = 4 * B * N * H * D * 2 + 3 * B * H * N * 4
        # the caching allocator rounds each block up; nothing of size N x N appears
        assert exact <= extra <= exact + 8 * 2 ** 20, (N, extra, exact)
        assert extra < 0.05 * B * H * N * N * 4, (N, extra)
        if per_token is not None:
            assert abs(extra / N - per_token) <= 0.02 * per_token, (N, extra / N, per_token)
        per_token = extra / N
        del x, o, lse, outs
