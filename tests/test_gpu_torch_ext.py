"""The torch extension _fhog_torch against flash_hog/_hip.py's Python wrappers.

Both call the same C-ABI entry points; the extension does the checks,
allocations and the call in C++. On the same inputs their outputs must be
bitwise equal, their errors the same (type and message), and the extension
must enqueue on torch's current stream like the wrappers do. The extension's
C++ autograd Functions (dot_product_attention's eager path) must give the
Python Functions' results bit for bit, refuse a third derivative as they do,
and give way to a swapped rule.
"""

from __future__ import annotations

import pytest
import torch

from helpers import make_inputs

pytestmark = pytest.mark.gpu

BF16, F16, F32 = torch.bfloat16, torch.float16, torch.float32


def _calls(x, o, lse, causal, scale):
    from flash_hog import _hip

    q, k, v, do, ddq, ddk, ddv = (x[n] for n in ("q", "k", "v", "do", "ddq", "ddk", "ddv"))
    return (_hip.attention_fwd(q, k, v, causal, scale)
            + _hip.attention_bwd(q, k, v, o, do, lse, causal, scale)
            + _hip.attention_bwdbwd(q, k, v, o, do, ddq, ddk, ddv, lse, causal, scale, return_stats=True)[:4]
            + _hip.attention_bwdbwd(q, k, v, o, do, ddq, ddk, ddv, lse, causal, scale, return_stats=True)[4])


# (id, batch, n_q, n_k, heads, kv_heads, head_dim, dtype, causal)
CASES = [
    ("bf16_causal", 2, 200, 200, 4, 4, 64, BF16, 1),
    ("f16_gqa_bottom_right_d128", 1, 96, 130, 4, 2, 128, F16, 2),
    ("f32_noncausal", 1, 77, 45, 2, 1, 64, F32, 0),
]


@pytest.mark.parametrize("case", CASES, ids=[c[0] for c in CASES])
def test_extension_equals_python_wrappers(case, cuda_device, monkeypatch):
    from flash_hog import _hip

    name, B, Nq, Nk, H, Hk, D, dtype, causal = case
    print(f"[case] torch ext {name}", flush=True)
    assert _hip.torch_ext() is not None, "the torch extension is not built"
    x = {n: t.to(cuda_device) for n, t in make_inputs(B, Nq, Nk, H, D, dtype, seed=3, kv_heads=Hk).items()}
    # a non-contiguous q: both paths copy it to a contiguous tensor first
    x["q"] = x["q"].transpose(1, 2).contiguous().transpose(1, 2)
    assert not x["q"].is_contiguous()
    scale = D ** -0.5
    o, lse = _hip.attention_fwd(x["q"], x["k"], x["v"], causal, scale)
    got = _calls(x, o, lse, causal, scale)
    torch.cuda.synchronize()
    monkeypatch.setattr(_hip, "torch_ext", lambda: None)
    want = _calls(x, o, lse, causal, scale)
    torch.cuda.synchronize()
    assert len(got) == len(want) == 13
    for i, (a, b) in enumerate(zip(got, want)):
        assert a.shape == b.shape and a.dtype == b.dtype and a.device == b.device, i
        assert torch.equal(a, b), i


def _error(fn, *args):
    with pytest.raises(Exception) as e:
        fn(*args)
    return e.type, str(e.value), getattr(e.value, "status", None)


def test_extension_errors_equal_python_wrappers(cuda_device, monkeypatch):
    """Shape and dtype mismatches (checked before the call) and an unsupported
    head dim (the C ABI's status, raised as FlashHogError) give the same error
    from both paths."""
    from flash_hog import _hip

    print("[case] torch ext errors", flush=True)
    mk = lambda *s, dt=BF16: torch.zeros(*s, dtype=dt, device=cuda_device)
    q, k = mk(1, 64, 2, 64), mk(1, 64, 2, 64)
    lse = torch.zeros(1, 2, 64, device=cuda_device)
    probes = [
        (_hip.attention_fwd, (q, k, mk(1, 63, 2, 64), 1, 0.125)),
        (_hip.attention_fwd, (q, k, mk(1, 64, 2, 64, dt=F16), 1, 0.125)),
        (_hip.attention_fwd, (q, mk(1, 64, 3, 64), mk(1, 64, 3, 64), 1, 0.125)),
        (_hip.attention_fwd, (mk(1, 64, 2, 96), mk(1, 64, 2, 96), mk(1, 64, 2, 96), 1, 0.125)),
        (_hip.attention_bwd, (q, k, k, q, q, torch.zeros(1, 2, 63, device=cuda_device), 1, 0.125)),
        (_hip.attention_bwdbwd, (q, k, k, q, q, q, k, mk(1, 64, 2, 32), lse, 1, 0.125)),
        (_hip.attention_bwdbwd, (q, k, k, q, q, q, k, k, lse, 7, 0.125)),
    ]
    got = [_error(fn, *a) for fn, a in probes]
    monkeypatch.setattr(_hip, "torch_ext", lambda: None)
    want = [_error(fn, *a) for fn, a in probes]
    assert got == want
    assert got[3][0] is _hip.FlashHogError and got[3][2] == _hip.FHOG_ERR_UNSUPPORTED
    assert got[6][0] is _hip.FlashHogError and got[6][2] == _hip.FHOG_ERR_INVALID_ARGUMENT


def test_extension_uses_the_current_stream(cuda_device):
    """Inputs written on a side stream and the call made on that stream: the
    kernels see the inputs (stream order), and the result equals a call on the
    default stream."""
    from flash_hog import _hip

    print("[case] torch ext current stream", flush=True)
    x = {n: t.to(cuda_device) for n, t in make_inputs(2, 256, 256, 2, 64, BF16, seed=8).items()}
    ref = _hip.attention_fwd(x["q"], x["k"], x["v"], 1, 0.125)
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    with torch.cuda.stream(side):
        q = torch.empty_like(x["q"])
        for _ in range(20):  # keep the side stream busy before the copy lands
            q.copy_(x["q"] * 0.0)
        q.copy_(x["q"])
        got = _hip.attention_fwd(q, x["k"], x["v"], 1, 0.125)
    side.synchronize()
    assert torch.equal(got[0], ref[0]) and torch.equal(got[1], ref[1])


# ------------------------------------------------- C++ autograd Functions

def _grads(x, causal, alignment, cot, tans, scale=None):
    import flash_hog

    x = [t.detach().requires_grad_(True) for t in x]
    out = flash_hog.dot_product_attention(*x, is_causal=causal, scale=scale, causal_alignment=alignment)
    g = torch.autograd.grad((out.float() * cot).sum(), x, create_graph=True)
    h = torch.autograd.grad(g, x, tans)
    return (out.detach(),) + tuple(t.detach() for t in g) + h


# (id, batch, n_q, n_k, heads, kv_heads, head_dim, dtype, is_causal, causal_alignment)
NATIVE_CASES = [
    ("bf16_causal", 2, 200, 200, 4, 4, 64, BF16, True, "top_left"),
    ("f16_gqa_bottom_right_d128", 1, 96, 130, 4, 2, 128, F16, True, "bottom_right"),
    ("f32_noncausal", 1, 77, 45, 2, 1, 64, F32, False, "top_left"),
    ("bf16_padded_d96", 1, 64, 64, 2, 2, 96, BF16, True, "top_left"),
]


@pytest.mark.parametrize("case", NATIVE_CASES, ids=[c[0] for c in NATIVE_CASES])
def test_native_autograd_equals_python_functions(case, cuda_device, monkeypatch):
    """dot_product_attention's C++ autograd Functions (eager, default rules)
    give the Python Functions' output, first gradients and Hessian-vector
    product bit for bit: the same kernels on the same operands."""
    from flash_hog.torch import attention as att

    name, B, Nq, Nk, H, Hk, D, dtype, causal, alignment = case
    print(f"[case] native autograd {name}", flush=True)
    x = {n: t.to(cuda_device) for n, t in make_inputs(B, Nq, Nk, H, D, dtype, seed=12, kv_heads=Hk).items()}
    qkv = (x["q"], x["k"], x["v"])
    cot = x["do"].float()
    tans = (x["ddq"], x["ddk"], x["ddv"])
    assert att._native_path(*qkv) is not None
    got = _grads(qkv, causal, alignment, cot, tans)
    torch.cuda.synchronize()
    monkeypatch.setattr(att, "_native_path", lambda *t: None)
    want = _grads(qkv, causal, alignment, cot, tans)
    torch.cuda.synchronize()
    for i, (a, b) in enumerate(zip(got, want)):
        assert a.shape == b.shape and a.dtype == b.dtype, i
        assert torch.equal(a, b), (name, i)


@pytest.mark.parametrize("native", [True, False], ids=["native", "python"])
def test_third_derivative_raises(native, cuda_device, monkeypatch):
    """The double backward is differentiable once, on either path: its results
    under create_graph carry a node that raises in a backward() through them,
    and grad() with respect to the inputs finds no path through them (the
    behaviour of torch's once_differentiable)."""
    import flash_hog
    from flash_hog.torch import attention as att

    print(f"[case] third derivative native={native}", flush=True)
    if not native:
        monkeypatch.setattr(att, "_native_path", lambda *t: None)
    x = {n: t.to(cuda_device) for n, t in make_inputs(1, 64, 64, 2, 64, BF16, seed=4).items()}
    qkv = [x[n].detach().requires_grad_(True) for n in ("q", "k", "v")]
    tans = [x[n].detach().requires_grad_(True) for n in ("ddq", "ddk", "ddv")]
    out = flash_hog.dot_product_attention(*qkv, is_causal=True)
    g = torch.autograd.grad(out.float().sum(), qkv, create_graph=True)
    h = torch.autograd.grad(g, qkv, tans, create_graph=True)
    assert all(t.requires_grad for t in h)
    third = torch.autograd.grad(sum(t.float().sum() for t in h), qkv + tans, allow_unused=True)
    assert all(t is None for t in third)
    h = torch.autograd.grad(g, qkv, tans, create_graph=True)
    with pytest.raises(RuntimeError, match="differentiate twice"):
        sum(t.float().sum() for t in h).backward()


def test_swapped_rule_takes_the_python_functions(cuda_device, monkeypatch):
    """A rule swapped in as a module attribute of _attention_impl is the one
    called: such calls leave the C++ Functions for the Python ones."""
    import flash_hog
    from flash_hog.torch import _attention_impl as attn_impl
    from flash_hog.torch import attention as att

    print("[case] swapped double-backward rule", flush=True)
    calls = []
    rule = attn_impl.dot_product_attention_bwd_rule_bwd_rule

    def counting(*args, **kwargs):
        calls.append(1)
        return rule(*args, **kwargs)

    monkeypatch.setattr(attn_impl, "dot_product_attention_bwd_rule_bwd_rule", counting)
    x = {n: t.to(cuda_device) for n, t in make_inputs(1, 64, 64, 2, 64, BF16, seed=6).items()}
    assert att._native_path(x["q"]) is None
    _grads((x["q"], x["k"], x["v"]), True, "top_left", x["do"].float(), (x["ddq"], x["ddk"], x["ddv"]))
    assert calls == [1]
    assert flash_hog.dot_product_attention is att.dot_product_attention
