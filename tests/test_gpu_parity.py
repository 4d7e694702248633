"""GPU parity of the HIP kernels against the CPU oracle (fp64) and the golden vectors.

Every kernel is called through the C ABI (flash_hog/_hip.py). Inputs are the
same seeded tensors for both sides; the oracle runs in float64 on the values
after rounding to the kernel's dtype. Tolerances (tests/helpers.py TOL):
max|a - r| / max|r| below 1e-3 for fp32, below 2e-2 for bf16 and fp16.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from helpers import DEGENERATE_FLOOR, TOL, default_scale, make_inputs, rel_err, stat_errs, to_np
from oracle import attention as ora

pytestmark = pytest.mark.gpu

F32, F16, BF16 = torch.float32, torch.float16, torch.bfloat16

# causal: 0 none, 1 top-left, 2 bottom-right (the C ABI's codes)
NONE, TL, BR = 0, 1, 2

# (id, batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal, qkv_scale)
CASES = [
    ("plumbing_f32_causal", 1, 256, 256, 2, 2, 64, F32, TL, 1.0),
    ("bf16_causal", 2, 256, 256, 3, 3, 64, BF16, TL, 1.0),
    ("bf16_noncausal", 2, 256, 256, 3, 3, 64, BF16, NONE, 1.0),
    ("f16_ragged_noncausal", 1, 1000, 1000, 2, 2, 64, F16, NONE, 0.5),
    ("bf16_ragged_causal", 1, 200, 200, 2, 2, 64, BF16, TL, 1.0),
    ("bf16_d128_causal", 1, 320, 320, 2, 2, 128, BF16, TL, 1.0),
    ("f16_d128_ragged_rect", 1, 100, 70, 1, 1, 128, F16, NONE, 1.0),
    ("bf16_rect_noncausal", 1, 128, 256, 2, 2, 64, BF16, NONE, 1.0),
    ("bf16_rect_causal", 1, 192, 256, 2, 2, 64, BF16, TL, 1.0),
    ("f32_noncausal_ragged", 2, 77, 45, 2, 2, 64, F32, NONE, 1.0),
    ("f32_single_token", 1, 1, 1, 1, 1, 64, F32, TL, 1.0),
    # grouped-query attention (query head h reads key/value head h // group)
    ("bf16_gqa4_causal", 2, 256, 256, 8, 2, 64, BF16, TL, 1.0),
    ("bf16_mqa_causal", 1, 256, 256, 4, 1, 64, BF16, TL, 1.0),
    ("f32_gqa3_causal_ragged", 1, 100, 100, 6, 2, 64, F32, TL, 1.0),
    ("f16_gqa2_d128_ragged_noncausal", 1, 200, 200, 4, 2, 128, F16, NONE, 0.5),
    # bottom-right causal (key j visible to query i iff j <= i + n_k - n_q)
    ("bf16_bottom_right_short_q", 1, 100, 300, 2, 2, 64, BF16, BR, 1.0),
    ("bf16_bottom_right_long_q", 1, 300, 100, 2, 2, 64, BF16, BR, 1.0),
    ("bf16_top_left_long_q", 1, 300, 100, 2, 2, 64, BF16, TL, 1.0),
    ("f32_bottom_right_gqa", 2, 64, 150, 4, 2, 64, F32, BR, 1.0),
    ("f16_bottom_right_mqa_d128", 1, 130, 257, 2, 1, 128, F16, BR, 1.0),
    ("bf16_bottom_right_square", 1, 256, 256, 2, 2, 64, BF16, BR, 1.0),
    # D = 256 (2-byte types)
    ("bf16_d256_causal", 1, 200, 200, 2, 2, 256, BF16, TL, 1.0),
    ("f16_d256_gqa2_ragged_noncausal", 2, 77, 130, 4, 2, 256, F16, NONE, 0.5),
    ("bf16_d256_bottom_right_long_q", 1, 150, 90, 2, 1, 256, BF16, BR, 1.0),
    # rows that see few keys (top-left causal, N_K << N_Q), and D = 256 with a large scale: the
    # fused stage 1's ddO subtracts dD O with dD summed over the bf16-rounded P ddS it multiplies
    ("bf16_causal_few_keys_gqa", 2, 298, 34, 2, 1, 64, BF16, TL, 1.0),
    # fp32 at D = 128
    ("f32_d128_causal", 1, 160, 160, 2, 2, 128, F32, TL, 1.0),
    ("f32_d128_gqa2_ragged_noncausal", 2, 77, 130, 4, 2, 128, F32, NONE, 1.0),
    ("f32_d128_bottom_right_long_q", 1, 200, 90, 2, 1, 128, F32, BR, 1.0),
]
IDS = [c[0] for c in CASES]

# Softmax scales other than the default 1/sqrt(D) (id, batch, n_q, n_k, heads,
# kv_heads, head_dim, dtype, causal, scale). Only a positive power-of-two scale
# lets the bf16 D = 64 kernels fold it into the resident operands; these cases
# run the general instances, and negative scales (the forward then takes its
# running maximum over the scaled logits' other end).
SCALE_CASES = [
    ("bf16_causal_scale_0.1", 2, 256, 256, 2, 2, 64, BF16, TL, 0.1),
    ("bf16_noncausal_ragged_scale_0.3", 1, 200, 200, 2, 2, 64, BF16, NONE, 0.3),
    ("bf16_causal_scale_-0.1", 1, 256, 256, 2, 2, 64, BF16, TL, -0.1),
    ("bf16_causal_scale_-0.125", 1, 192, 192, 2, 2, 64, BF16, TL, -0.125),
    ("f16_noncausal_ragged_scale_-0.2", 1, 150, 150, 2, 2, 64, F16, NONE, -0.2),
    ("f16_d128_bottom_right_scale_-0.05", 1, 100, 160, 2, 1, 128, F16, BR, -0.05),
    # power-of-two scales at D = 128 (both stages fold them into their resident operands)
    ("bf16_d128_causal_scale_0.125", 1, 300, 300, 4, 2, 128, BF16, TL, 0.125),
    ("bf16_d128_noncausal_ragged_scale_0.0625", 2, 150, 230, 2, 2, 128, BF16, NONE, 0.0625),
    ("f32_causal_scale_-0.125", 1, 96, 96, 2, 2, 64, F32, TL, -0.125),
    ("f32_d128_causal_scale_0.3", 1, 100, 100, 2, 2, 128, F32, TL, 0.3),
    ("bf16_d256_causal_scale_0.0625", 1, 100, 100, 2, 2, 256, BF16, TL, 0.0625),
    ("bf16_d256_noncausal_scale_-0.05", 1, 100, 120, 2, 2, 256, BF16, NONE, -0.05),
    ("bf16_d256_noncausal_scale_0.199", 2, 266, 239, 2, 2, 256, BF16, NONE, 0.199),
]
SCALE_IDS = [c[0] for c in SCALE_CASES]


def _lse_err(lse, lse_ref):
    """max |L - L_ref| over rows that see a key, relative to max(1, |L_ref|);
    rows that see no key must hold +inf on both sides."""
    got, ref = to_np(lse), np.asarray(lse_ref)
    empty = np.isposinf(ref)
    assert np.array_equal(np.isposinf(got), empty), "rows without keys must have L = +inf"
    if empty.all():
        return 0.0
    return float(np.max(np.abs(got[~empty] - ref[~empty])) / max(1.0, np.max(np.abs(ref[~empty]))))


def _announce(*what):
    print("[case]", *what, flush=True)


def _oracle_residual(x, scale, causal, dtype):
    """O (rounded to dtype) and L (fp32) from the fp64 oracle forward."""
    o, lse = ora.attn_fwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), scale, causal)
    return torch.from_numpy(o).to(dtype), torch.from_numpy(lse).float()


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_fwd_matches_oracle(case, cuda_device):
    name, B, Nq, Nk, H, Hk, D, dtype, causal, qs = case
    _announce("fwd", name)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=11, qkv_scale=qs, kv_heads=Hk)
    scale = default_scale(D)
    from flash_hog import _hip

    o, lse = _hip.attention_fwd(x["q"].to(cuda_device), x["k"].to(cuda_device), x["v"].to(cuda_device),
                                causal, scale)
    torch.cuda.synchronize()
    o_ref, lse_ref = ora.attn_fwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), scale, causal)
    assert rel_err(o, o_ref, DEGENERATE_FLOOR) < TOL[dtype]
    assert _lse_err(lse, lse_ref) < 1e-3


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_bwd_matches_oracle(case, cuda_device):
    name, B, Nq, Nk, H, Hk, D, dtype, causal, qs = case
    _announce("bwd", name)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=23, qkv_scale=qs, kv_heads=Hk)
    scale = default_scale(D)
    o, lse = _oracle_residual(x, scale, causal, dtype)
    from flash_hog import _hip

    g = lambda t: t.to(cuda_device)
    dq, dk, dv, delta = _hip.attention_bwd(g(x["q"]), g(x["k"]), g(x["v"]), g(o), g(x["do"]), g(lse),
                                           causal, scale)
    torch.cuda.synchronize()
    ref = ora.attn_bwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), to_np(o), to_np(x["do"]),
                       to_np(lse), scale, causal)
    for got, want, label in zip((dq, dk, dv, delta), ref, ("dq", "dk", "dv", "D")):
        err = rel_err(got, want, DEGENERATE_FLOOR)
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"


@pytest.mark.parametrize("case", CASES, ids=IDS)
def test_bwdbwd_matches_oracle(case, cuda_device):
    name, B, Nq, Nk, H, Hk, D, dtype, causal, qs = case
    _announce("bwdbwd", name)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=37, qkv_scale=qs, kv_heads=Hk)
    scale = default_scale(D)
    o, lse = _oracle_residual(x, scale, causal, dtype)
    from flash_hog import _hip

    g = lambda t: t.to(cuda_device)
    dq2, dk2, dv2, ddo, stats = _hip.attention_bwdbwd(
        g(x["q"]), g(x["k"]), g(x["v"]), g(o), g(x["do"]), g(x["ddq"]), g(x["ddk"]), g(x["ddv"]), g(lse),
        causal, scale, return_stats=True)
    torch.cuda.synchronize()
    ref = ora.attn_bwd_bwd_stats(*(to_np(x[n]) for n in ("q", "k", "v")), to_np(o), to_np(x["do"]),
                                 *(to_np(x[n]) for n in ("ddq", "ddk", "ddv")), to_np(lse), scale, causal,
                                 return_stats=True)
    got = (dq2, dk2, dv2, ddo) + tuple(stats)
    for a, r, label in zip(got[:4], ref[:4], ("dq2", "dk2", "dv2", "ddo")):
        err = rel_err(a, r, DEGENERATE_FLOOR)
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"
    for err, label in zip(stat_errs(got[4:], ref[4:]), ("D", "dD", "B")):
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"
    for a, label in zip(got, ("dq2", "dk2", "dv2", "ddo", "D", "dD", "B")):
        assert torch.isfinite(torch.as_tensor(a)).all(), label


@pytest.mark.parametrize("case", SCALE_CASES, ids=SCALE_IDS)
def test_all_kernels_other_scales(case, cuda_device):
    """Forward, first backward and double backward against the oracle at
    non-default and negative softmax scales."""
    name, B, Nq, Nk, H, Hk, D, dtype, causal, scale = case
    _announce("scale", name)
    from flash_hog import _hip

    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=53, kv_heads=Hk)
    g = lambda t: t.to(cuda_device)
    o_k, lse_k = _hip.attention_fwd(g(x["q"]), g(x["k"]), g(x["v"]), causal, scale)
    torch.cuda.synchronize()
    o_ref, lse_ref = ora.attn_fwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), scale, causal)
    assert rel_err(o_k, o_ref, DEGENERATE_FLOOR) < TOL[dtype], "O"
    assert _lse_err(lse_k, lse_ref) < 1e-3, "L"

    o, lse = _oracle_residual(x, scale, causal, dtype)
    got = _hip.attention_bwd(g(x["q"]), g(x["k"]), g(x["v"]), g(o), g(x["do"]), g(lse), causal, scale)
    torch.cuda.synchronize()
    ref = ora.attn_bwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), to_np(o), to_np(x["do"]), to_np(lse),
                       scale, causal)
    for a, r, label in zip(got, ref, ("dq", "dk", "dv", "D")):
        err = rel_err(a, r, DEGENERATE_FLOOR)
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"

    dq2, dk2, dv2, ddo, stats = _hip.attention_bwdbwd(
        g(x["q"]), g(x["k"]), g(x["v"]), g(o), g(x["do"]), g(x["ddq"]), g(x["ddk"]), g(x["ddv"]), g(lse),
        causal, scale, return_stats=True)
    torch.cuda.synchronize()
    ref = ora.attn_bwd_bwd_stats(*(to_np(x[n]) for n in ("q", "k", "v")), to_np(o), to_np(x["do"]),
                                 *(to_np(x[n]) for n in ("ddq", "ddk", "ddv")), to_np(lse), scale, causal,
                                 return_stats=True)
    for a, r, label in zip((dq2, dk2, dv2, ddo), ref[:4], ("dq2", "dk2", "dv2", "ddo")):
        err = rel_err(a, r, DEGENERATE_FLOOR)
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"
    for err, label in zip(stat_errs(tuple(stats), ref[4:]), ("D", "dD", "B")):
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"


# Problems with rows that see exactly one key (id, batch, n_q, n_k, heads,
# kv_heads, head_dim, dtype, causal). N_K = 1 makes every row such a row; a
# causal mask makes the first row that sees a key one (row -coff).
SINGLE_KEY_CASES = [
    ("bf16_nk1_mqa", 1, 70, 1, 4, 1, 64, BF16, NONE),
    ("bf16_d128_nk1_bottom_right", 2, 40, 1, 2, 2, 128, BF16, BR),
    ("f16_nk1_top_left_gqa", 1, 33, 1, 4, 2, 64, F16, TL),
    ("f32_nk1_mqa", 1, 50, 1, 4, 1, 64, F32, NONE),
    ("f32_causal_mqa_first_row", 1, 100, 100, 4, 1, 64, F32, TL),
    ("bf16_d128_bottom_right_first_row", 1, 130, 100, 2, 1, 128, BF16, BR),
]


@pytest.mark.parametrize("case", SINGLE_KEY_CASES, ids=[c[0] for c in SINGLE_KEY_CASES])
def test_single_key_rows_are_exact(case, cuda_device):
    """A row that sees one key has a constant softmax (P = 1 whatever Q, K,
    V), so the double backward is exact there: dQ2 = 0 and ddO = ddV of the
    key, and the row adds nothing to dK2 and dV2 (all zero when N_K = 1). The
    kernels' fp32 sums only cancel to rounding of the row statistics, which
    for fp32 inputs can exceed the oracle tolerance measured against an
    exact zero; they keep such rows exact instead. Every output is also
    compared with the oracle."""
    name, B, Nq, Nk, H, Hk, D, dtype, causal = case
    _announce("single key", name)
    from flash_hog import _hip

    scale = default_scale(D)
    x = make_inputs(B, Nq, Nk, H, D, dtype, seed=61, kv_heads=Hk)
    o, lse = _oracle_residual(x, scale, causal, dtype)
    g = lambda t: t.to(cuda_device)
    dq2, dk2, dv2, ddo, stats = _hip.attention_bwdbwd(
        g(x["q"]), g(x["k"]), g(x["v"]), g(o), g(x["do"]), g(x["ddq"]), g(x["ddk"]), g(x["ddv"]), g(lse),
        causal, scale, return_stats=True)
    torch.cuda.synchronize()
    ref = ora.attn_bwd_bwd_stats(*(to_np(x[n]) for n in ("q", "k", "v")), to_np(o), to_np(x["do"]),
                                 *(to_np(x[n]) for n in ("ddq", "ddk", "ddv")), to_np(lse), scale, causal,
                                 return_stats=True)
    for a, r, label in zip((dq2, dk2, dv2, ddo), ref[:4], ("dq2", "dk2", "dv2", "ddo")):
        err = rel_err(a, r, DEGENERATE_FLOOR)
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"
    for err, label in zip(stat_errs(tuple(stats), ref[4:]), ("D", "dD", "B")):
        assert err < TOL[dtype], f"{label}: rel err {err:.3e}"

    coff = {NONE: 0, TL: 0, BR: Nk - Nq}[causal]
    seen = [Nk if causal == NONE else max(0, min(Nk, i + coff + 1)) for i in range(Nq)]
    rows = [i for i in range(Nq) if seen[i] == 1]
    assert rows, "the case must hold a row that sees one key"
    dq2, ddo = dq2.cpu(), ddo.cpu()
    assert torch.count_nonzero(dq2[:, rows]) == 0, "dQ2 of single-key rows"
    # the key such a row sees is key 0; query head h reads key/value head h // (H / Hk)
    want = x["ddv"][:, 0].repeat_interleave(H // Hk, dim=1)[:, None].expand(B, len(rows), H, D)
    got = ddo[:, rows]
    if dtype == F32:
        assert rel_err(got, want) < 1e-5, "ddO of single-key rows"
    else:
        assert torch.equal(got, want.to(dtype)), "ddO of single-key rows"
    if Nk == 1:
        assert torch.count_nonzero(dk2) == 0 and torch.count_nonzero(dv2) == 0, "dK2 and dV2 with one key"


def _golden():
    import pathlib

    path = pathlib.Path(__file__).resolve().parent / "golden" / "test_data.npz"
    return dict(np.load(path))


@pytest.mark.parametrize("dtype", [F32, BF16], ids=["f32", "bf16"])
def test_bwdbwd_golden_vectors(dtype, cuda_device):
    """The reference's test_data.zip (non-causal, 128 x 256 x 64, scale 1/8)
    through the HIP double backward, with the fixture's own O and L."""
    _announce("golden", dtype)
    z = _golden()
    t = lambda n: torch.from_numpy(z[n])[None, :, None, :].to(dtype).to(cuda_device)
    lse = torch.from_numpy(z["L"])[None, None, :].float().to(cuda_device)
    from flash_hog import _hip

    outs = _hip.attention_bwdbwd(t("q"), t("k"), t("v"), t("o"), t("do"), t("ddq"), t("ddk"), t("ddv"), lse,
                                 False, 0.125)
    torch.cuda.synchronize()
    for a, n in zip(outs, ("dq2", "dk2", "dv2", "ddo")):
        err = rel_err(a[0, :, 0, :], z[n])
        # the fixture itself carries bf16-level error (its L is a bf16-precision logsumexp)
        assert err < 2e-2, f"{n}: rel err {err:.3e}"


def test_gpu_reference_matches_oracle(cuda_device):
    """Pins the fp32 GPU checkers used at full size (forward, first backward,
    double backward) against the fp64 oracle."""
    import gpu_reference

    _announce("gpu_reference pin")
    x = make_inputs(1, 160, 160, 2, 64, F32, seed=5)
    scale = default_scale(64)
    o, lse = _oracle_residual(x, scale, True, F32)
    g = lambda t: t.to(cuda_device)
    o_g, l_g = gpu_reference.fwd(g(x["q"]), g(x["k"]), g(x["v"]), scale, True)
    o_r, l_r = ora.attn_fwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), scale, True)
    assert rel_err(o_g, o_r) < 1e-4
    assert _lse_err(l_g, l_r) < 1e-5
    got = gpu_reference.bwd(g(x["q"]), g(x["k"]), g(x["v"]), g(o), g(x["do"]), g(lse), scale, True)
    ref = ora.attn_bwd(to_np(x["q"]), to_np(x["k"]), to_np(x["v"]), to_np(o), to_np(x["do"]), to_np(lse),
                       scale, True)
    for a, r in zip(got, ref):
        assert rel_err(a, r) < 1e-4
    got = gpu_reference.bwdbwd(*(g(x[n]) for n in ("q", "k", "v")), g(o), g(x["do"]),
                               *(g(x[n]) for n in ("ddq", "ddk", "ddv")), g(lse), scale, True)
    ref = ora.attn_bwd_bwd_stats(*(to_np(x[n]) for n in ("q", "k", "v")), to_np(o), to_np(x["do"]),
                                 *(to_np(x[n]) for n in ("ddq", "ddk", "ddv")), to_np(lse), scale, True)
    for a, r in zip(got, ref):
        assert rel_err(a, r) < 1e-4



@pytest.mark.parametrize("causal", [True, False], ids=["causal", "noncausal"])
def test_gpu_reference_chunked(causal, cuda_device):
    """The row-chunked closed forms (used by bench.py's HVP tables at long
    sequences) equal the unchunked ones pinned above, with a ragged last chunk."""
    import gpu_reference

    _announce(f"gpu_reference chunked causal={causal}")
    x = make_inputs(1, 600, 600, 1, 64, F32, seed=9)
    scale = default_scale(64)
    h = {n: t[0, :, 0, :].contiguous().to(cuda_device) for n, t in x.items()}
    o, lse = gpu_reference.fwd_head(h["q"], h["k"], h["v"], scale, causal)
    o_c, lse_c = gpu_reference.fwd_head_chunked(h["q"], h["k"], h["v"], scale, causal, rows=128)
    assert rel_err(o_c, o) < 1e-5 and rel_err(lse_c, lse) < 1e-6
    args = (h["q"], h["k"], h["v"], o, h["do"], h["ddq"], h["ddk"], h["ddv"], lse, scale, causal)
    ref = gpu_reference.bwdbwd_head(*args)
    got = gpu_reference.bwdbwd_head_chunked(*args, rows=128)
    for a, r in zip(got, ref):
        assert rel_err(a, r) < 1e-5