"""The forward, first backward and double backward at the full sizes of the
benchmark configurations.

Each configuration runs through the C ABI at its real shape. Parity is checked
against tests/gpu_reference.py (the closed forms in fp32 on the GPU, one
(batch, head) at a time, on the same dtype-rounded inputs; each is pinned to
the fp64 oracle in test_gpu_parity.py), on every head; at 32768 tokens the
double backward's reference is evaluated in blocks of query rows. The residual (O, L) that the backward
kernels consume comes from gpu_reference.fwd (O rounded to the input dtype),
never from this library's forward, so an error of the forward cannot cancel
out of a backward comparison. Properties that hold at any size are checked
too:

- the rows of dS (first backward) and of dS, dS2, ddP (double backward) sum
  to zero, so the key-sums of dK, dK2 and dV2 vanish, and the rows of P sum
  to one, so the key-sum of dV equals the query-sum of dO (per batch, head
  and column);
- the double backward is linear in the cotangents (ddQ, ddK, ddV), so doubling
  them doubles every output (a power-of-two scale is exact in floating point;
  only values that cross the subnormal range may round differently);
- causally, rows [0, M) of O, L, dQ, dQ2 and ddO depend only on the first M
  keys, so a length-N run and a length-M run agree on them bit for bit;
- the extra device memory of a call (outputs plus three fp32 row vectors) grows
  linearly in N; no (N, N) buffer is allocated.

Tolerance: max|a - r| / max|r| < 2e-2 for bf16 and fp16 inputs (the parity bar
for 2-byte runs against an fp32 reference); L to 1e-3 of max(1, |L|).
"""

from __future__ import annotations

import math

import pytest
import torch

import gpu_reference
from helpers import make_inputs, rel_err

pytestmark = pytest.mark.gpu

TOL_2BYTE = 2e-2
TOL_LSE = 1e-3

BF16, F16 = torch.bfloat16, torch.float16

# name -> batch, seq, heads, head_dim, dtype, causal, q/k/v scale, seed, heads checked (None = all)
CONFIGS = {
    "standard_b4_n2048_h16_d64_bf16_causal": (4, 2048, 16, 64, BF16, True, 1.0, 101, None),
    "long_b2_n8192_h16_d128_bf16_causal": (2, 8192, 16, 128, BF16, True, 1.0, 202, None),
    "ragged_b8_n1000_h12_d64_f16_noncausal": (8, 1000, 12, 64, F16, False, 0.5, 303, None),
}


def _announce(*what):
    print("[case]", *what, flush=True)


def _all_heads(B, H):
    return [(b, h) for b in range(B) for h in range(H)]


def _setup(B, N, H, D, dtype, causal, qkv_scale, device, seed):
    """Seeded inputs and the reference residual: O (fp32 forward, rounded to
    dtype) and L (fp32) on every head."""
    x = make_inputs(B, N, N, H, D, dtype, seed=seed, qkv_scale=qkv_scale, device=device)
    scale = 1.0 / math.sqrt(D)
    o32, lse = gpu_reference.fwd(x["q"], x["k"], x["v"], scale, causal)
    return x, o32.to(dtype), lse, scale


def _lse_err(a, r):
    return ((a.float() - r.float()).abs().max() / r.float().abs().max().clamp(min=1.0)).item()


def _bwdbwd(x, o, lse, causal, scale, mul=1.0):
    from flash_hog import _hip

    return _hip.attention_bwdbwd(x["q"], x["k"], x["v"], o, x["do"], x["ddq"] * mul, x["ddk"] * mul,
                                 x["ddv"] * mul, lse, causal, scale)


def _head(t, b, h):
    return t[b:b + 1, :, h:h + 1, :]


def _check_fwd(x, o, lse, scale, causal, heads):
    o_ref, l_ref = gpu_reference.fwd(x["q"], x["k"], x["v"], scale, causal, heads=heads)
    worst_o = max(rel_err(_head(o, b, h), _head(o_ref, b, h)) for b, h in heads)
    worst_l = max(_lse_err(lse[b, h], l_ref[b, h]) for b, h in heads)
    assert worst_o < TOL_2BYTE, f"O: rel err {worst_o:.3e}"
    assert worst_l < TOL_LSE, f"L: err {worst_l:.3e}"


def _check_bwd(x, o, lse, got, scale, causal, heads):
    ref = gpu_reference.bwd(x["q"], x["k"], x["v"], o, x["do"], lse, scale, causal, heads=heads)
    for label, a, r in zip(("dq", "dk", "dv"), got[:3], ref[:3]):
        err = max(rel_err(_head(a, b, h), _head(r, b, h)) for b, h in heads)
        assert err < TOL_2BYTE, f"{label}: rel err {err:.3e}"
    err = max(rel_err(got[3][b, h], ref[3][b, h]) for b, h in heads)
    assert err < TOL_2BYTE, f"D: rel err {err:.3e}"


def _check_bwd_sums(x, got):
    """sum over keys of dK is zero; sum over keys of dV equals sum over queries of dO."""
    dk, dv = got[1].float(), got[2].float()
    s, mag = dk.sum(dim=1).abs().max().item(), dk.abs().sum(dim=1).max().item()
    assert s <= TOL_2BYTE * mag, f"dk: |sum over keys| {s:.3e} vs magnitude {mag:.3e}"
    err = (dv.sum(dim=1) - x["do"].float().sum(dim=1)).abs().max().item()
    mag = dv.abs().sum(dim=1).max().item()
    assert err <= TOL_2BYTE * mag, f"dv: key-sum minus query-sum of dO {err:.3e} vs magnitude {mag:.3e}"


def _check_heads(x, o, lse, outs, scale, causal, heads):
    """gpu_reference on the listed (batch, head) pairs, against the kernel's outputs."""
    names = ("dq2", "dk2", "dv2", "ddo")
    worst = {n: 0.0 for n in names}
    for b, h in heads:
        sl = lambda t: _head(t, b, h)
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


@pytest.mark.parametrize("name", list(CONFIGS))
def test_fwd_full_size(name, cuda_device):
    from flash_hog import _hip

    B, N, H, D, dtype, causal, qs, seed, heads = CONFIGS[name]
    _announce("fwd", name)
    x = make_inputs(B, N, N, H, D, dtype, seed=seed, qkv_scale=qs, device=cuda_device)
    scale = 1.0 / math.sqrt(D)
    o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
    torch.cuda.synchronize()
    _check_fwd(x, o, lse, scale, causal, heads or _all_heads(B, H))


@pytest.mark.parametrize("name", list(CONFIGS))
def test_bwd_full_size(name, cuda_device):
    from flash_hog import _hip

    B, N, H, D, dtype, causal, qs, seed, heads = CONFIGS[name]
    _announce("bwd", name)
    x, o, lse, scale = _setup(B, N, H, D, dtype, causal, qs, cuda_device, seed)
    got = _hip.attention_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, causal, scale)
    torch.cuda.synchronize()
    _check_bwd(x, o, lse, got, scale, causal, heads or _all_heads(B, H))
    _check_bwd_sums(x, got)


def test_standard_b4_n2048_h16_d64_bf16_causal(cuda_device):
    _announce("bwdbwd config standard B4 N2048 H16 D64 bf16 causal")
    B, N, H, D = 4, 2048, 16, 64
    x, o, lse, scale = _setup(B, N, H, D, BF16, True, 1.0, cuda_device, seed=101)
    outs = _bwdbwd(x, o, lse, True, scale)
    torch.cuda.synchronize()
    _check_heads(x, o, lse, outs, scale, True, _all_heads(B, H))
    _check_key_sums(outs)
    doubled = _bwdbwd(x, o, lse, True, scale, mul=2.0)
    for a, a2 in zip(outs, doubled):
        assert rel_err(a2, a.float() * 2) < 1e-6


def test_long_b2_n8192_h16_d128_bf16_causal(cuda_device):
    _announce("bwdbwd config long B2 N8192 H16 D128 bf16 causal")
    B, N, H, D = 2, 8192, 16, 128
    x, o, lse, scale = _setup(B, N, H, D, BF16, True, 1.0, cuda_device, seed=202)
    outs = _bwdbwd(x, o, lse, True, scale)
    torch.cuda.synchronize()
    _check_heads(x, o, lse, outs, scale, True, _all_heads(B, H))
    _check_key_sums(outs)


def test_ragged_b8_n1000_h12_d64_f16_noncausal(cuda_device):
    _announce("bwdbwd config ragged B8 N1000 H12 D64 fp16 non-causal")
    B, N, H, D = 8, 1000, 12, 64
    x, o, lse, scale = _setup(B, N, H, D, F16, False, 0.5, cuda_device, seed=303)
    outs = _bwdbwd(x, o, lse, False, scale)
    torch.cuda.synchronize()
    _check_heads(x, o, lse, outs, scale, False, _all_heads(B, H))
    _check_key_sums(outs)


def test_very_long_b1_n32768_h8_d64_bf16_causal(cuda_device):
    """The full 32768-token run of all three kernels, checked on a 4096-token
    slice. The forward's O and L rows [0, 4096), the first backward's dQ and D
    rows and the double backward's dQ2 and ddO rows equal those of 4096-token
    runs on the same inputs bit for bit; the 4096-token runs match
    gpu_reference on every head; the full runs satisfy the key-sum invariants.
    The full double backward is also compared, on every head and all four
    outputs, with gpu_reference's row-chunked closed form
    (bwdbwd_head_chunked, pinned to the unchunked one by
    test_gpu_parity.py::test_gpu_reference_chunked): dK2 and dV2 of keys
    below 4096 sum over all 32768 queries, which no 4096-token run sees."""
    from flash_hog import _hip

    _announce("config very long B1 N32768 H8 D64 bf16 causal")
    B, N, H, D, M = 1, 32768, 8, 64, 4096
    x, o, lse, scale = _setup(B, N, H, D, BF16, True, 1.0, cuda_device, seed=404)
    xs = {n: t[:, :M].contiguous() for n, t in x.items()}
    os_, ls_ = o[:, :M].contiguous(), lse[:, :, :M].contiguous()
    heads = _all_heads(B, H)

    _announce("  forward")
    o_k, l_k = _hip.attention_fwd(x["q"], x["k"], x["v"], True, scale)
    o_s, l_s = _hip.attention_fwd(xs["q"], xs["k"], xs["v"], True, scale)
    torch.cuda.synchronize()
    assert torch.equal(o_k[:, :M], o_s), "O prefix"
    assert torch.equal(l_k[:, :, :M], l_s), "L prefix"
    assert _lse_err(l_k, lse) < TOL_LSE, "L of the full run"
    assert rel_err(o_k, o) < TOL_2BYTE, "O of the full run"
    _check_fwd(xs, o_s, l_s, scale, True, heads)
    del o_k, l_k, o_s, l_s

    _announce("  first backward")
    full = _hip.attention_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, True, scale)
    short = _hip.attention_bwd(xs["q"], xs["k"], xs["v"], os_, xs["do"], ls_, True, scale)
    torch.cuda.synchronize()
    assert torch.equal(full[0][:, :M], short[0]), "dq prefix"
    assert torch.equal(full[3][:, :, :M], short[3]), "D prefix"
    assert all(torch.isfinite(t).all() for t in full)
    _check_bwd_sums(x, full)
    _check_bwd(xs, os_, ls_, short, scale, True, heads)
    del full, short

    _announce("  double backward")
    outs = _bwdbwd(x, o, lse, True, scale)
    torch.cuda.synchronize()
    assert all(torch.isfinite(t).all() for t in outs)
    _check_key_sums(outs)
    worst = {n: 0.0 for n in ("dq2", "dk2", "dv2", "ddo")}
    for h in range(H):
        _announce(f"  double backward, head {h}, against the row-chunked reference")
        sl = lambda t: t[0, :, h, :].float().contiguous()
        ref = gpu_reference.bwdbwd_head_chunked(
            sl(x["q"]), sl(x["k"]), sl(x["v"]), sl(o), sl(x["do"]), sl(x["ddq"]), sl(x["ddk"]), sl(x["ddv"]),
            lse[0, h].contiguous(), scale, True, rows=4096)
        for n, a, r in zip(worst, outs, ref):
            worst[n] = max(worst[n], rel_err(a[0, :, h, :], r))
        del ref
    print("  worst rel err over heads:", {n: f"{e:.2e}" for n, e in worst.items()}, flush=True)
    for n, e in worst.items():
        assert e < TOL_2BYTE, f"{n} of the full run: rel err {e:.3e}"
    short = _bwdbwd(xs, os_, ls_, True, scale)
    torch.cuda.synchronize()
    assert torch.equal(outs[0][:, :M], short[0]), "dq2 prefix"
    assert torch.equal(outs[3][:, :M], short[3]), "ddo prefix"
    _check_heads(xs, os_, ls_, short, scale, True, heads)


def test_peak_memory_is_linear_in_n(cuda_device):
    """Extra device memory of one call (B1 H8 D64 bf16 causal) from N = 4096
    to 32768: the four outputs and the three fp32 row vectors, linear in N."""
    from flash_hog import _hip

    B, H, D = 1, 8, 64
    per_token = None
    for N in (4096, 8192, 16384, 32768):
        _announce("peak memory N", N)
        x = make_inputs(B, N, N, H, D, BF16, seed=7, device=cuda_device)
        scale = 1.0 / math.sqrt(D)
        o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], True, scale)
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
