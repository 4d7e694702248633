"""Grad-of-grad through the public front-end, mirroring the reference's tests.

tests/test_jax_fhog.py:56-62 builds vjp(f) with f(Q, K, V, dO) = vjp(attn)(dO)
and compares it with XLA autodiff of jax.nn.dot_product_attention
(make_reference_dpa_bwd_bwd, :26-34). Here the same composition runs through
flash_hog.dot_product_attention (HIP forward, first backward and double
backward) and is compared with the torch-CPU autodiff oracle in float64.
"""

from __future__ import annotations

import pytest
import torch

from helpers import TOL, default_scale, make_inputs, rel_err
from oracle import autodiff

pytestmark = pytest.mark.gpu


def fhog_bwd_bwd(q, k, v, do, ddq, ddk, ddv, is_causal, scale, **kw):
    import flash_hog

    q, k, v, do = (t.detach().requires_grad_(True) for t in (q, k, v, do))
    out = flash_hog.dot_product_attention(q, k, v, is_causal=is_causal, scale=scale, **kw)
    dq, dk, dv = torch.autograd.grad(out, (q, k, v), do, create_graph=True)
    return torch.autograd.grad((dq, dk, dv), (q, k, v, do), (ddq, ddk, ddv)), (out, dq, dk, dv)


@pytest.mark.parametrize("is_causal", [True, False], ids=["causal", "noncausal"])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
def test_backward_backward_single(is_causal, dtype, cuda_device):
    print("[case] frontend grad-of-grad", dtype, is_causal, flush=True)
    x = make_inputs(2, 192, 192, 4, 64, dtype, seed=42)
    scale = default_scale(64)
    dev = {n: t.to(cuda_device) for n, t in x.items()}
    (dq2, dk2, dv2, ddo), (out, dq, dk, dv) = fhog_bwd_bwd(
        dev["q"], dev["k"], dev["v"], dev["do"], dev["ddq"], dev["ddk"], dev["ddv"], is_causal, scale)
    torch.cuda.synchronize()
    c = {n: t.double() for n, t in x.items()}
    ref2 = autodiff.double_vjp(c["q"], c["k"], c["v"], c["do"], c["ddq"], c["ddk"], c["ddv"], scale, is_causal)
    ref1 = autodiff.first_vjp(c["q"], c["k"], c["v"], c["do"], scale, is_causal)
    ref_out = autodiff.attention(c["q"], c["k"], c["v"], scale, is_causal)
    assert rel_err(out, ref_out) < TOL[dtype]
    for a, r, n in zip((dq, dk, dv), ref1, ("dq", "dk", "dv")):
        assert rel_err(a, r) < TOL[dtype], n
    for a, r, n in zip((dq2, dk2, dv2, ddo), ref2, ("dq2", "dk2", "dv2", "ddo")):
        assert rel_err(a, r) < TOL[dtype], n


@pytest.mark.parametrize("head_dim,dtype,is_causal", [
    (32, torch.bfloat16, True), (80, torch.bfloat16, False), (96, torch.float16, True),
    (16, torch.bfloat16, True), (40, torch.float32, True), (96, torch.float32, False), (160, torch.bfloat16, True),
], ids=["d32_bf16_causal", "d80_bf16", "d96_f16_causal", "d16_bf16_causal", "d40_f32_causal", "d96_f32",
        "d160_bf16_causal"])
def test_padded_head_dims(head_dim, dtype, is_causal, cuda_device):
    """Head dims the kernels do not take natively (the reference's kernel has no
    head-dim limit, flash_hog/jax/_pallas_gpu_kernel.py:80-101) run zero-padded
    to 64, 128 or 256: forward, first and second derivatives against the fp64
    autodiff oracle, at the unpadded head dim's default scale."""
    print("[case] frontend padded head dim", head_dim, dtype, is_causal, flush=True)
    x = make_inputs(2, 150, 150, 2, head_dim, dtype, seed=61)
    scale = default_scale(head_dim)
    dev = {n: t.to(cuda_device) for n, t in x.items()}
    (dq2, dk2, dv2, ddo), (out, dq, dk, dv) = fhog_bwd_bwd(
        dev["q"], dev["k"], dev["v"], dev["do"], dev["ddq"], dev["ddk"], dev["ddv"], is_causal, None)
    torch.cuda.synchronize()
    assert out.shape == dev["q"].shape and dq2.shape == dev["q"].shape
    c = {n: t.double() for n, t in x.items()}
    ref2 = autodiff.double_vjp(c["q"], c["k"], c["v"], c["do"], c["ddq"], c["ddk"], c["ddv"], scale, is_causal)
    ref1 = autodiff.first_vjp(c["q"], c["k"], c["v"], c["do"], scale, is_causal)
    ref_out = autodiff.attention(c["q"], c["k"], c["v"], scale, is_causal)
    assert rel_err(out, ref_out) < TOL[dtype]
    for a, r, n in zip((dq, dk, dv), ref1, ("dq", "dk", "dv")):
        assert rel_err(a, r) < TOL[dtype], n
    for a, r, n in zip((dq2, dk2, dv2, ddo), ref2, ("dq2", "dk2", "dv2", "ddo")):
        assert rel_err(a, r) < TOL[dtype], n


def test_unbatched_inputs(cuda_device):
    """(T, N, H) inputs get a batch axis added and removed (attention.py:39-47)."""
    import flash_hog

    print("[case] frontend unbatched", flush=True)
    x = make_inputs(1, 64, 64, 2, 64, torch.bfloat16, seed=3)
    q, k, v = (x[n][0].to(cuda_device) for n in ("q", "k", "v"))
    out = flash_hog.dot_product_attention(q, k, v, is_causal=True)
    out_b = flash_hog.dot_product_attention(q[None], k[None], v[None], is_causal=True)
    assert out.shape == q.shape
    assert torch.equal(out, out_b[0])


def test_hvp_matches_double_vjp(cuda_device):
    """A Hessian-vector product of a scalar loss runs the double backward."""
    import flash_hog

    print("[case] frontend hvp", flush=True)
    x = make_inputs(1, 128, 128, 2, 64, torch.float32, seed=9)
    q, k, v = (x[n].to(cuda_device).requires_grad_(True) for n in ("q", "k", "v"))
    w = x["do"].to(cuda_device)
    u = (x["ddq"].to(cuda_device), x["ddk"].to(cuda_device), x["ddv"].to(cuda_device))
    loss = (flash_hog.dot_product_attention(q, k, v, is_causal=True) * w).sum()
    g = torch.autograd.grad(loss, (q, k, v), create_graph=True)
    hvp = torch.autograd.grad(g, (q, k, v), u)
    torch.cuda.synchronize()
    c = {n: t.double() for n, t in x.items()}
    ref = autodiff.double_vjp(c["q"], c["k"], c["v"], c["do"], c["ddq"], c["ddk"], c["ddv"], 0.125, True)
    for a, r in zip(hvp, ref[:3]):
        assert rel_err(a, r) < 1e-3


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32], ids=["bf16", "f32"])
@pytest.mark.parametrize("nq,nk,heads,kv_heads,alignment", [
    (96, 160, 4, 2, "bottom_right"),
    (160, 96, 6, 2, "bottom_right"),
    (128, 128, 8, 1, "top_left"),
], ids=["br_short_q_gqa2", "br_long_q_gqa3", "mqa_top_left"])
def test_backward_backward_gqa_and_alignment(nq, nk, heads, kv_heads, alignment, dtype, cuda_device):
    """Grad-of-grad with grouped key/value heads and either causal alignment,
    against the fp64 autograd oracle with the same grouping and mask."""
    print("[case] frontend grad-of-grad", dtype, nq, nk, heads, kv_heads, alignment, flush=True)
    x = make_inputs(2, nq, nk, heads, 64, dtype, seed=44, kv_heads=kv_heads)
    scale = default_scale(64)
    code = 2 if alignment == "bottom_right" else 1
    dev = {n: t.to(cuda_device) for n, t in x.items()}
    (dq2, dk2, dv2, ddo), (out, dq, dk, dv) = fhog_bwd_bwd(
        dev["q"], dev["k"], dev["v"], dev["do"], dev["ddq"], dev["ddk"], dev["ddv"], True, scale,
        causal_alignment=alignment)
    torch.cuda.synchronize()
    c = {n: t.double() for n, t in x.items()}
    ref2 = autodiff.double_vjp(c["q"], c["k"], c["v"], c["do"], c["ddq"], c["ddk"], c["ddv"], scale, code)
    ref1 = autodiff.first_vjp(c["q"], c["k"], c["v"], c["do"], scale, code)
    ref_out = autodiff.attention(c["q"], c["k"], c["v"], scale, code)
    if nq > nk:  # rows without keys: the oracle's softmax gives NaN there, the kernels zeros
        e = nq - nk
        assert torch.all(out[:, :e] == 0) and torch.all(dq[:, :e] == 0)
        assert torch.all(dq2[:, :e] == 0) and torch.all(ddo[:, :e] == 0)
        ref_out = ref_out.nan_to_num(0.0)
        # key-side and remaining rows: the square problem made of the last nk queries
        sq = {n: (t[:, e:] if n in ("q", "do", "ddq") else t) for n, t in c.items()}
        ref2 = autodiff.double_vjp(sq["q"], sq["k"], sq["v"], sq["do"], sq["ddq"], sq["ddk"], sq["ddv"], scale, 1)
        ref1 = autodiff.first_vjp(sq["q"], sq["k"], sq["v"], sq["do"], scale, 1)
        dq, dq2, ddo = dq[:, e:], dq2[:, e:], ddo[:, e:]
    assert rel_err(out, ref_out) < TOL[dtype]
    for a, r, n in zip((dq, dk, dv), ref1, ("dq", "dk", "dv")):
        assert rel_err(a, r) < TOL[dtype], n
    for a, r, n in zip((dq2, dk2, dv2, ddo), ref2, ("dq2", "dk2", "dv2", "ddo")):
        assert rel_err(a, r) < TOL[dtype], n


def test_vmap_hvp_equals_folded_batch(cuda_device):
    """torch.func.vmap of a per-example Hessian-vector product folds the mapped
    axis into the batch axis (one kernel call per rule), so it equals, bit for
    bit, the batched computation on the folded tensors."""
    import flash_hog

    print("[case] frontend vmap hvp", flush=True)
    V, B, N, H, Hk, D = 3, 2, 128, 4, 2, 64
    x = make_inputs(V * B, N, N, H, D, torch.bfloat16, seed=51, kv_heads=Hk)
    dev = {n: t.to(cuda_device) for n, t in x.items()}

    def loss(q, k, v, w):
        return (flash_hog.dot_product_attention(q, k, v, is_causal=True).float() * w.float()).sum()

    def g_dot_u(q, k, v, w, uq, uk, uv):
        gr = torch.func.grad(loss, argnums=(0, 1, 2))(q, k, v, w)
        return sum((a.float() * b.float()).sum() for a, b in zip(gr, (uq, uk, uv)))

    hvp = torch.func.grad(g_dot_u, argnums=(0, 1, 2))
    unfold = lambda t: t.unflatten(0, (V, B))
    args = [dev[n] for n in ("q", "k", "v", "do", "ddq", "ddk", "ddv")]
    mapped = torch.func.vmap(hvp)(*(unfold(t) for t in args))
    folded = hvp(*args)
    torch.cuda.synchronize()
    for a, b in zip(mapped, folded):
        assert torch.equal(a.flatten(0, 1), b)
    # an unmapped key/value pair is broadcast along the mapped axis
    kv = dict(in_dims=(0, None, None, 0))
    out = torch.func.vmap(lambda q, k, v, w: flash_hog.dot_product_attention(q, k, v, is_causal=True), **kv)(
        unfold(dev["q"]), dev["k"][:B], dev["v"][:B], unfold(dev["do"]))
    ref = flash_hog.dot_product_attention(dev["q"], dev["k"][:B].repeat(V, 1, 1, 1), dev["v"][:B].repeat(V, 1, 1, 1),
                                          is_causal=True)
    assert torch.equal(out.flatten(0, 1), ref)


@pytest.mark.parametrize("kw,expect", [
    (dict(is_causal=True, seq_len=2048, head_dim=64, num_q_heads=16, num_kv_heads=16), True),
    (dict(is_causal=False, seq_len=1000, head_dim=64, num_q_heads=12, num_kv_heads=4, dtype=torch.float16), True),
    (dict(is_causal=True, seq_len=200, head_dim=128, num_q_heads=4, num_kv_heads=4, kv_seq_len=300,
          causal_alignment="bottom_right"), True),
    (dict(is_causal=True, seq_len=256, head_dim=96, num_q_heads=2, num_kv_heads=2), True),
    (dict(is_causal=True, seq_len=256, head_dim=160, num_q_heads=2, num_kv_heads=2), True),
    (dict(is_causal=True, seq_len=256, head_dim=320, num_q_heads=2, num_kv_heads=2), False),
    (dict(is_causal=True, seq_len=256, head_dim=128, num_q_heads=2, num_kv_heads=2, dtype=torch.float32), True),
    (dict(is_causal=True, seq_len=256, head_dim=192, num_q_heads=2, num_kv_heads=2, dtype=torch.float32), False),
    (dict(is_causal=True, seq_len=256, head_dim=64, num_q_heads=3, num_kv_heads=2), False),
], ids=["bench", "gqa_f16", "d128_br", "d96_padded", "d160_padded", "d320", "f32_d128", "f32_d192", "bad_groups"])
def test_supported_agrees_with_a_call(kw, expect, cuda_device):
    """flash_hog.supported (the reference's _tk_gpu.py:70-80 query) says True
    exactly where the front-end's double backward runs."""
    import flash_hog

    assert flash_hog.supported(**kw) is expect
    dtype = kw.get("dtype", torch.bfloat16)
    gen = torch.Generator().manual_seed(1)
    B, T, S = 1, kw["seq_len"], kw.get("kv_seq_len", kw["seq_len"])
    mk = lambda n, h: torch.randn((B, n, h, kw["head_dim"]), generator=gen).to(cuda_device, dtype)
    q, k, v = mk(T, kw["num_q_heads"]), mk(S, kw["num_kv_heads"]), mk(S, kw["num_kv_heads"])
    do, ddq, ddk, ddv = torch.randn_like(q), torch.randn_like(q), torch.randn_like(k), torch.randn_like(v)
    align = kw.get("causal_alignment", "top_left")
    if expect:
        fhog_bwd_bwd(q, k, v, do, ddq, ddk, ddv, kw["is_causal"], None, causal_alignment=align)
        torch.cuda.synchronize()
    else:
        with pytest.raises((ValueError, RuntimeError)):
            fhog_bwd_bwd(q, k, v, do, ddq, ddk, ddv, kw["is_causal"], None, causal_alignment=align)


def test_torch_compile_matches_eager(cuda_device):
    """A torch.compile'd (aot_eager backend, whole graph) forward and gradient
    run the same kernels as eager: outputs and gradients bitwise equal."""
    import flash_hog

    print("[case] frontend torch.compile", flush=True)
    x = {n: t.to(cuda_device) for n, t in make_inputs(2, 192, 192, 4, 64, torch.bfloat16, seed=21, kv_heads=2).items()}

    def loss(q, k, v):
        out = flash_hog.dot_product_attention(q, k, v, is_causal=True)
        return (out.float() * x["do"].float()).sum(), out

    results = []
    for fn in (loss, torch.compile(loss, backend="aot_eager", fullgraph=True)):
        q, k, v = (x[n].clone().requires_grad_(True) for n in ("q", "k", "v"))
        val, out = fn(q, k, v)
        results.append((out.detach(), *torch.autograd.grad(val, (q, k, v))))
    torch.cuda.synchronize()
    for a, b in zip(*results):
        assert torch.equal(a, b)
