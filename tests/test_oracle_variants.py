"""Pins the oracle's grouped-query heads and bottom-right causal mask.

Grouped heads: query head h uses key/value head h // G (G = H_q / H_kv), the
grouping "(kv_heads group)" of flash_hog/jax/_pallas_gpu_kernel.py:106-107,
which is also torch SDPA's enable_gqa grouping (repeat_interleave); the
key-side gradients sum over each group (_pallas_gpu_kernel.py:333-370).

Bottom-right causal: key j visible to query i iff j <= i + N_K - N_Q
(flash_hog/_jax_refs/jax_impl.py:104-109), torch's causal_lower_right bias.
Queries that see no key (N_Q > N_K) are defined here to give zeros; the
reference's softmax (and torch's SDPA) gives NaN for them.

Every check compares the oracle with a library routine (SDPA, autograd) or a
structural identity, and the mutation tests confirm that a plausible mistake
in the head mapping or the mask offset is caught.
"""

from __future__ import annotations

import inspect
import warnings

import numpy as np
import pytest
import torch

from oracle import attention as ora
from oracle import autodiff


def rand(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape)


def inputs(B, Nq, Nk, H, Hk, D, seed=0):
    names = ("q", "k", "v", "do", "ddq", "ddk", "ddv")
    out = {}
    for i, n in enumerate(names):
        shape = (B, Nq, H, D) if n in ("q", "do", "ddq") else (B, Nk, Hk, D)
        out[n] = rand(shape, seed + i)
    return out


def full(x, scale, causal):
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], scale, causal)
    outs = ora.attn_bwd_bwd_stats(x["q"], x["k"], x["v"], o, x["do"], x["ddq"], x["ddk"], x["ddv"], lse,
                                  scale, causal)
    return o, lse, outs


def t(x):
    return torch.from_numpy(x)


def bhtd(x):
    return t(x).permute(0, 2, 1, 3)


def sdpa(q, k, v, scale, causal):
    """torch SDPA (fp64 CPU) on (B, T, H, D) arrays; causal 1 top-left, 2 bottom-right."""
    from torch.nn.attention.bias import causal_lower_right

    tq, tk, tv = bhtd(q), bhtd(k), bhtd(v)
    gqa = tq.shape[1] != tk.shape[1]
    if causal == 2:
        with warnings.catch_warnings():
            warnings.simplefilter("ignore")
            mask = causal_lower_right(tq.shape[2], tk.shape[2])
        if gqa:  # the bias object does not combine with enable_gqa; repeat explicitly
            G = tq.shape[1] // tk.shape[1]
            tk, tv = tk.repeat_interleave(G, 1), tv.repeat_interleave(G, 1)
        out = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, attn_mask=mask, scale=scale)
    else:
        out = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=bool(causal), scale=scale,
                                                               enable_gqa=gqa)
    return out.permute(0, 2, 1, 3)


# ------------------------------------------------------------ grouped heads

@pytest.mark.parametrize("causal", [0, 1, 2])
def test_gqa_forward_matches_sdpa(causal):
    x = inputs(2, 13, 13, 6, 2, 8, seed=11)
    o, _ = ora.attn_fwd(x["q"], x["k"], x["v"], 0.3, causal)
    assert ora.rel_err(o, sdpa(x["q"], x["k"], x["v"], 0.3, causal).numpy()) < 1e-12


@pytest.mark.parametrize("causal", [0, 1])
def test_gqa_first_backward_matches_sdpa_autograd(causal):
    """Autograd through SDPA's enable_gqa sums dK, dV over each group."""
    x = inputs(1, 11, 15, 4, 2, 8, seed=12)
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], 0.4, causal)
    got = ora.attn_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, 0.4, causal)[:3]
    tq, tk, tv = (bhtd(x[n]).requires_grad_(True) for n in ("q", "k", "v"))
    out = torch.nn.functional.scaled_dot_product_attention(tq, tk, tv, is_causal=bool(causal), scale=0.4,
                                                           enable_gqa=True)
    ref = torch.autograd.grad(out, (tq, tk, tv), bhtd(x["do"]))
    for a, r in zip(got, ref):
        assert ora.rel_err(a, r.permute(0, 2, 1, 3).numpy()) < 1e-12


@pytest.mark.parametrize("causal", [0, 1, 2])
def test_gqa_double_backward_matches_autograd(causal):
    x = inputs(2, 9, 14, 6, 3, 8, seed=13)
    _, _, ref = full(x, 0.35, causal)
    tt = {n: t(v) for n, v in x.items()}
    got = autodiff.double_vjp(tt["q"], tt["k"], tt["v"], tt["do"], tt["ddq"], tt["ddk"], tt["ddv"], 0.35, causal)
    for a, r in zip(got, ref):
        assert ora.rel_err(a.numpy(), r) < 1e-11


def test_autodiff_gqa_attention_matches_sdpa():
    """The autograd oracle's head repetition is SDPA's enable_gqa grouping."""
    x = inputs(1, 10, 10, 8, 2, 8, seed=14)
    got = autodiff.attention(t(x["q"]), t(x["k"]), t(x["v"]), 0.3, 1)
    assert ora.rel_err(got.numpy(), sdpa(x["q"], x["k"], x["v"], 0.3, 1).numpy()) < 1e-12


def test_gqa_equals_repeated_heads():
    """Grouped problem == ungrouped problem with k-side tensors repeated per
    group; the grouped key-side gradients are the per-group sums."""
    G, Hk = 3, 2
    x = inputs(1, 12, 12, G * Hk, Hk, 8, seed=15)
    rep = dict(x)
    for n in ("k", "v", "ddk", "ddv"):
        rep[n] = np.repeat(x[n], G, axis=2)
    o_g, l_g, (dq2_g, dk2_g, dv2_g, ddo_g) = full(x, 0.3, 1)
    o_r, l_r, (dq2_r, dk2_r, dv2_r, ddo_r) = full(rep, 0.3, 1)
    assert np.allclose(o_g, o_r, rtol=0, atol=1e-13) and np.allclose(l_g, l_r, rtol=0, atol=1e-13)
    assert np.allclose(dq2_g, dq2_r, rtol=0, atol=1e-12) and np.allclose(ddo_g, ddo_r, rtol=0, atol=1e-12)
    fold = lambda a: a.reshape(a.shape[0], a.shape[1], Hk, G, a.shape[3]).sum(axis=3)
    assert np.allclose(dk2_g, fold(dk2_r), rtol=0, atol=1e-12)
    assert np.allclose(dv2_g, fold(dv2_r), rtol=0, atol=1e-12)


# ------------------------------------------------------ bottom-right causal

@pytest.mark.parametrize("nq,nk", [(7, 19), (16, 16), (19, 19)])
def test_bottom_right_forward_matches_sdpa(nq, nk):
    x = inputs(2, nq, nk, 2, 2, 8, seed=16)
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], 0.3, 2)
    assert ora.rel_err(o, sdpa(x["q"], x["k"], x["v"], 0.3, 2).numpy()) < 1e-12
    s = torch.einsum("bqhd,bkhd->bhqk", t(x["q"]), t(x["k"])) * 0.3
    s = s.masked_fill(~t(ora.causal_mask(nq, nk, 2)), float("-inf"))
    assert np.max(np.abs(lse - torch.logsumexp(s, -1).numpy())) < 1e-12


def test_bottom_right_is_top_left_when_square():
    x = inputs(1, 17, 17, 2, 2, 8, seed=17)
    a = full(x, 0.3, 1)
    b = full(x, 0.3, 2)
    for u, w in zip((a[0], a[1]) + tuple(a[2]), (b[0], b[1]) + tuple(b[2])):
        assert np.array_equal(u, w)


def test_bottom_right_double_backward_matches_autograd():
    x = inputs(2, 8, 21, 2, 2, 8, seed=18)
    _, _, ref = full(x, 0.3, 2)
    tt = {n: t(v) for n, v in x.items()}
    got = autodiff.double_vjp(tt["q"], tt["k"], tt["v"], tt["do"], tt["ddq"], tt["ddk"], tt["ddv"], 0.3, 2)
    for a, r in zip(got, ref):
        assert ora.rel_err(a.numpy(), r) < 1e-11


def test_bottom_right_first_backward_matches_autograd():
    x = inputs(1, 6, 13, 2, 2, 8, seed=19)
    o, lse = ora.attn_fwd(x["q"], x["k"], x["v"], 0.3, 2)
    got = ora.attn_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, 0.3, 2)[:3]
    ref = autodiff.first_vjp(t(x["q"]), t(x["k"]), t(x["v"]), t(x["do"]), 0.3, 2)
    for a, r in zip(got, ref):
        assert ora.rel_err(a, r.numpy()) < 1e-12


def test_bottom_right_rows_without_keys():
    """N_Q > N_K: the first N_Q - N_K queries see no key. Their O, dQ2 and ddO
    rows are zero and L is +inf; the remaining rows and every key-side output
    equal those of the square problem made of the last N_K queries."""
    nq, nk = 20, 12
    x = inputs(1, nq, nk, 2, 2, 8, seed=20)
    o, lse, (dq2, dk2, dv2, ddo) = full(x, 0.3, 2)
    e = nq - nk
    assert np.all(o[:, :e] == 0) and np.all(np.isposinf(lse[:, :, :e]))
    assert np.all(dq2[:, :e] == 0) and np.all(ddo[:, :e] == 0)
    sq = {n: (v[:, e:] if n in ("q", "do", "ddq") else v) for n, v in x.items()}
    o_s, lse_s, (dq2_s, dk2_s, dv2_s, ddo_s) = full(sq, 0.3, 1)
    assert np.allclose(o[:, e:], o_s, rtol=0, atol=1e-13)
    assert np.allclose(lse[:, :, e:], lse_s, rtol=0, atol=1e-13)
    for a, r in ((dq2[:, e:], dq2_s), (ddo[:, e:], ddo_s), (dk2, dk2_s), (dv2, dv2_s)):
        assert np.allclose(a, r, rtol=0, atol=1e-12)
    d = ora.attn_bwd(x["q"], x["k"], x["v"], o, x["do"], lse, 0.3, 2)
    assert np.all(d[0][:, :e] == 0)


def test_pair_count_matches_masks():
    for nq, nk in ((5, 3), (3, 5), (7, 7), (20, 12), (12, 20)):
        for causal in (1, 2):
            assert int(ora.causal_mask(nq, nk, causal).sum()) == autodiff.unmasked_pairs(nq, nk, causal)


# ------------------------------------------------------------ mutation tests

def _with_mutant(fn_name, src_from, src_to):
    src = inspect.getsource(getattr(ora, fn_name))
    assert src_from in src, src_from
    ns = dict(vars(ora))
    exec(src.replace(src_from, src_to), ns)
    return ns[fn_name]


def test_sdpa_check_rejects_wrong_head_mapping():
    """h % H_kv (interleaved groups) instead of h // G is caught by SDPA's grouping."""
    mut = _with_mutant("attn_fwd", "K[b, h // G], V[b, h // G]", "K[b, h % K.shape[1]], V[b, h % K.shape[1]]")
    x = inputs(1, 9, 9, 6, 2, 8, seed=21)
    o, _ = mut(x["q"], x["k"], x["v"], 0.3, 1)
    assert ora.rel_err(o, sdpa(x["q"], x["k"], x["v"], 0.3, 1).numpy()) > 1e-2


def test_sdpa_check_rejects_wrong_mask_offset():
    """A bottom-right offset of the wrong sign is caught by causal_lower_right."""
    mut = _with_mutant("causal_mask", "n_k - n_q if", "n_q - n_k if")
    orig = ora.causal_mask
    x = inputs(1, 7, 19, 2, 2, 8, seed=22)
    try:
        ora.causal_mask = mut
        o, _ = ora.attn_fwd(x["q"], x["k"], x["v"], 0.3, 2)
    finally:
        ora.causal_mask = orig
    o = np.nan_to_num(o, nan=1e3)
    assert ora.rel_err(o, sdpa(x["q"], x["k"], x["v"], 0.3, 2).numpy()) > 1e-2
