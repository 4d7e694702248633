"""Pins the CPU oracle (oracle/attention.py) before the GPU tests compare against it.

Each oracle function is checked against something other than its own formula:
the reference's golden vectors, finite differences, torch autograd (a library
routine), closed-form special cases and invariants. The mutation tests at the
end plant plausible mistakes in a copy of the oracle and confirm that the
checks reject them.
"""

from __future__ import annotations

import inspect
import pathlib

import numpy as np
import pytest
import torch

from oracle import attention as ora
from oracle import autodiff

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden" / "test_data.npz"


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def inputs(B, Nq, Nk, H, D, seed=0):
    names = ("q", "k", "v", "do", "ddq", "ddk", "ddv")
    out = {}
    for i, n in enumerate(names):
        shape = (B, Nq, H, D) if n in ("q", "do", "ddq") else (B, Nk, H, D)
        out[n] = rand(shape, seed + i)
    return out


def full(x, scale, causal, head=None):
    """Oracle double backward with O, L from the oracle forward."""
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], scale, causal)
    return ora.attn_bwd_bwd_stats(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"], lse,
                                  scale, causal, return_stats=True)


def first_order(q, k, v, do, scale, causal):
    o, lse = ora.attn_fwd(q, k, v, scale, causal)
    return ora.attn_bwd(q, k, v, o, do, lse, scale, causal)[:3]


# ---------------------------------------------------------------- golden KAT

def test_golden_vectors():
    """flash_hog/_jax_refs/jax_impl.py:594-654 wrote test_data.zip from
    attn_bwd_bwd_stats under bf16 matmul precision; the fp64 restatement with
    the fixture's own O and L reproduces it to bf16-level error."""
    z = dict(np.load(GOLDEN))
    t = lambda n: z[n][None, :, None, :].astype(np.float64)
    outs = ora.attn_bwd_bwd_stats(t("q"), t("k"), t("v"), t("o"), t("do"), t("ddq"), t("ddk"), t("ddv"),
                                  z["L"][None, None, :].astype(np.float64), 0.125, False)
    errs = {n: ora.rel_err(a[0, :, 0, :], z[n]) for a, n in zip(outs, ("dq2", "dk2", "dv2", "ddo"))}
    assert max(errs.values()) < 1e-2, errs
    # the fixture agrees far better with the restatement than with a perturbed one
    assert min(errs.values()) < 5e-3, errs


def test_golden_fixture_is_self_consistent():
    """The fixture's O and L are the forward of its q, k, v (up to bf16 rounding)."""
    z = dict(np.load(GOLDEN))
    t = lambda n: z[n][None, :, None, :].astype(np.float64)
    o, lse = ora.attn_fwd(t("q"), t("k"), t("v"), 0.125, False)
    assert ora.rel_err(o[0, :, 0, :], z["o"]) < 1e-2
    assert np.max(np.abs(lse[0, 0] - z["L"])) < 2e-2


# ----------------------------------------------------------- finite differences

def _fd_check(bwdbwd_fn, scale, causal, seed=1, eps=1e-6):
    """<(ddQ, ddK, ddV), J t> by central differences of the first-order backward
    equals <(dQ2, dK2, dV2, ddO), t> for a random direction t."""
    B, Nq, Nk, H, D = 1, 11, 13, 2, 8
    x = inputs(B, Nq, Nk, H, D, seed)
    t = {n: rand(x[n].shape, 100 + i) for i, n in enumerate(("q", "k", "v", "do"))}
    outs = bwdbwd_fn(x, scale, causal)
    lhs = sum(np.sum(outs[i] * t[n]) for i, n in enumerate(("q", "k", "v", "do")))

    def f(sign):
        args = [x[n] + sign * eps * t[n] for n in ("q", "k", "v", "do")]
        return first_order(*args, scale, causal)

    plus, minus = f(+1), f(-1)
    rhs = sum(np.sum((p - m) / (2 * eps) * x[n]) for p, m, n in zip(plus, minus, ("ddq", "ddk", "ddv")))
    return abs(lhs - rhs) / max(abs(rhs), 1e-30)


@pytest.mark.parametrize("causal", [False, True])
def test_finite_differences(causal):
    err = _fd_check(lambda x, s, c: full(x, s, c)[:4], 0.35, causal)
    assert err < 1e-7, err


# ------------------------------------------------------------ library routines

@pytest.mark.parametrize("causal", [False, True])
def test_matches_torch_autograd_double_vjp(causal):
    """Closed form == torch autograd of the reference's XLA oracle composition
    (tests/test_jax_fhog.py:26-34), in float64."""
    x = inputs(2, 17, 17, 3, 16, seed=4)
    scale = 0.25
    ref = full(x, scale, causal)
    tt = {n: torch.from_numpy(v) for n, v in x.items()}
    got = autodiff.double_vjp(tt["q"], tt["k"], tt["v"], tt["do"], tt["ddq"], tt["ddk"], tt["ddv"], scale, causal)
    for a, r in zip(got, ref[:4]):
        assert ora.rel_err(a.numpy(), r) < 1e-11


def test_rectangular_matches_autograd():
    x = inputs(1, 9, 21, 2, 8, seed=8)
    ref = full(x, 0.3, False)
    tt = {n: torch.from_numpy(v) for n, v in x.items()}
    got = autodiff.double_vjp(tt["q"], tt["k"], tt["v"], tt["do"], tt["ddq"], tt["ddk"], tt["ddv"], 0.3, False)
    for a, r in zip(got, ref[:4]):
        assert ora.rel_err(a.numpy(), r) < 1e-11


@pytest.mark.parametrize("causal", [False, True])
def test_forward_matches_torch(causal):
    x = inputs(2, 19, 19, 2, 16, seed=2)
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], 0.25, causal)
    tq, tk, tv = (torch.from_numpy(x[n]).permute(0, 2, 1, 3) for n in ("q", "k", "v"))
    ref = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=causal, scale=0.25)
    assert ora.rel_err(o, ref.permute(0, 2, 1, 3).numpy()) < 1e-12
    s = torch.einsum("bhqd,bhkd->bhqk", tq, tk) * 0.25
    if causal:
        s = s.masked_fill(~torch.ones(19, 19, dtype=torch.bool).tril(), float("-inf"))
    assert np.max(np.abs(lse - torch.logsumexp(s, -1).numpy())) < 1e-12


def test_forward_causal_first_row_and_row_sums():
    x = inputs(1, 12, 12, 1, 8, seed=3)
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], 0.5, True)
    assert np.allclose(o[0, 0, 0], x["v"][0, 0, 0])
    assert np.isclose(lse[0, 0, 0], 0.5 * x["q"][0, 0, 0] @ x["k"][0, 0, 0])
    p = np.exp(ora._scores(x["q"][0, :, 0], x["k"][0, :, 0], 0.5, True) - lse[0, 0][:, None])
    assert np.allclose(p.sum(-1), 1.0)


@pytest.mark.parametrize("causal", [False, True])
def test_first_backward_matches_autograd(causal):
    x = inputs(1, 14, 14, 2, 8, seed=6)
    got = first_order(x["q"], x["k"], x["v"], x["do"], 0.4, causal)
    tt = {n: torch.from_numpy(v) for n, v in x.items()}
    ref = autodiff.first_vjp(tt["q"], tt["k"], tt["v"], tt["do"], 0.4, causal)
    for a, r in zip(got, ref):
        assert ora.rel_err(a, r.numpy()) < 1e-12
    # rows of dS sum to zero, so the key-sum of dK vanishes
    assert np.max(np.abs(got[1].sum(axis=1))) < 1e-12 * np.max(np.abs(got[1])) * 14


# --------------------------------------------------- invariants, special cases

@pytest.mark.parametrize("causal", [False, True])
def test_key_sums_of_dk2_and_dv2_vanish(causal):
    """Rows of dS, dS2 and ddP sum to zero, so sum over keys of dK2 and dV2 is 0."""
    x = inputs(1, 24, 24, 2, 8, seed=9)
    dq2, dk2, dv2, ddo = full(x, 0.3, causal)[:4]
    assert np.max(np.abs(dk2.sum(axis=1))) < 1e-12 * np.max(np.abs(dk2)) * 24
    assert np.max(np.abs(dv2.sum(axis=1))) < 1e-12 * np.max(np.abs(dv2)) * 24


@pytest.mark.parametrize("causal", [False, True])
def test_special_case_reduces_to_first_order(causal):
    """ddQ = ddK = 0: dV2 = 0, ddO = P ddV, (dQ2, dK2) = first-order (dQ, dK)
    of attention with V replaced by ddV."""
    x = inputs(1, 15, 15, 2, 8, seed=12)
    x["ddq"] = np.zeros_like(x["ddq"])
    x["ddk"] = np.zeros_like(x["ddk"])
    dq2, dk2, dv2, ddo = full(x, 0.3, causal)[:4]
    assert np.max(np.abs(dv2)) < 1e-14
    p_ddv, _ = ora.attn_fwd(x["q"], x["k"], x["ddv"], 0.3, causal)
    assert ora.rel_err(ddo, p_ddv) < 1e-12
    dq, dk, _ = first_order(x["q"], x["k"], x["ddv"], x["do"], 0.3, causal)
    assert ora.rel_err(dq2, dq) < 1e-12
    assert ora.rel_err(dk2, dk) < 1e-12


def test_linear_in_cotangents():
    x = inputs(1, 10, 10, 1, 8, seed=13)
    y = dict(x)
    for i, n in enumerate(("ddq", "ddk", "ddv")):
        y[n] = rand(x[n].shape, 50 + i)
    z = dict(x)
    for n in ("ddq", "ddk", "ddv"):
        z[n] = 2.0 * x[n] - 3.0 * y[n]
    fx, fy, fz = (full(w, 0.3, True)[:4] for w in (x, y, z))
    for a, b, c in zip(fx, fy, fz):
        assert ora.rel_err(c, 2.0 * a - 3.0 * b) < 1e-12


def test_causal_prefix_property():
    """Rows [0, M) of dQ2 and ddO depend only on the first M tokens."""
    x = inputs(1, 20, 20, 1, 8, seed=14)
    M = 11
    xm = {n: v[:, :M] for n, v in x.items()}
    a, b = full(x, 0.3, True), full(xm, 0.3, True)
    assert ora.rel_err(a[0][:, :M], b[0]) < 1e-12
    assert ora.rel_err(a[3][:, :M], b[3]) < 1e-12


def test_row_statistics():
    """D = rowsum(O dO) equals rowsum(P dP); dD and B follow from the outputs:
    sum_j P_ij dP2_ij = B_i with dP2 from the definitions."""
    x = inputs(1, 16, 16, 1, 8, seed=15)
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], 0.3, True)
    *_, d, dd, bst = ora.attn_bwd_bwd_stats(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"],
                                            lse, 0.3, True, return_stats=True)
    q, k, v, do = (x[n][0, :, 0] for n in ("q", "k", "v", "do"))
    p = np.exp(ora._scores(q, k, 0.3, True) - lse[0, 0][:, None])
    assert np.allclose(d[0, 0], np.sum(p * (do @ v.T), -1))
    dds = 0.3 * (x["ddq"][0, :, 0] @ k.T + q @ x["ddk"][0, :, 0].T)
    assert np.allclose(dd[0, 0], np.sum(p * dds, -1))
    # B via the identity used by the fused first sweep
    dp = do @ v.T
    dpa = do @ x["ddv"][0, :, 0].T
    r1, r2, r3 = np.sum(dpa * p, -1), np.sum(dp * p, -1), np.sum(dp * dds * p, -1)
    assert np.allclose(bst[0, 0], r1 - dd[0, 0] * r2 - d[0, 0] * dd[0, 0] + r3)


def test_unmasked_pair_count():
    assert autodiff.unmasked_pairs(2048, 2048, True) == 2048 * 2049 // 2
    assert autodiff.unmasked_pairs(1000, 1000, False) == 1000 * 1000
    assert autodiff.unmasked_pairs(5, 3, True) == 6 + 2 * 3
    m = ora.causal_mask(5, 3)
    assert int(m.sum()) == autodiff.unmasked_pairs(5, 3, True)
    flops = autodiff.bwdbwd_algorithmic_flops(4, 16, 2048, 2048, 64, True)
    assert abs(flops / 1e9 - 206.3) < 0.1


# -------------------------------------------------------------- mutation tests

MUTATIONS = [
    ("- dds * d[:, None]", "+ dds * d[:, None]"),        # sign of the ddS*D term
    ("dp * dds", "dp * dp"),                              # wrong operand
    ("ds.T @ ddq + ds2.T @ q", "ds.T @ ddq"),             # dropped term
    ("p @ ddv + ddp @ v", "p @ ddv - ddp @ v"),          # sign of a product
    ("ddp.T @ do", "ddp.T @ ddq"),                        # transposed/wrong operand
]


def _mutant(src_from, src_to):
    src = inspect.getsource(ora.bwd_bwd_head)
    assert src_from in src, src_from
    ns = dict(vars(ora))
    exec(src.replace(src_from, src_to), ns)
    mutated = ns["bwd_bwd_head"]

    def fn(x, scale, causal):
        o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], scale, causal)
        orig = ora.bwd_bwd_head
        try:
            ora.bwd_bwd_head = mutated
            return ora.attn_bwd_bwd_stats(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"],
                                          lse, scale, causal)
        finally:
            ora.bwd_bwd_head = orig

    return fn


@pytest.mark.parametrize("mutation", MUTATIONS, ids=[m[1] for m in MUTATIONS])
def test_finite_difference_check_rejects_mutants(mutation):
    err = _fd_check(_mutant(*mutation), 0.35, True)
    assert err > 1e-3, f"mutation {mutation} not detected (err {err:.2e})"


def test_golden_check_rejects_mutants():
    z = dict(np.load(GOLDEN))
    t = lambda n: z[n][None, :, None, :].astype(np.float64)
    lse = z["L"][None, None, :].astype(np.float64)
    for frm, to in MUTATIONS:
        src = inspect.getsource(ora.bwd_bwd_head).replace(frm, to)
        ns = dict(vars(ora))
        exec(src, ns)
        outs = ns["bwd_bwd_head"](*(t(n)[0, :, 0] for n in ("q", "k", "v", "o", "do", "ddq", "ddk", "ddv")),
                                  lse[0, 0], 0.125, False)[:4]
        errs = [ora.rel_err(a, z[n]) for a, n in zip(outs, ("dq2", "dk2", "dv2", "ddo"))]
        assert max(errs) > 2e-2, (frm, to, errs)
