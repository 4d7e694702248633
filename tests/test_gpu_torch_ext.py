"""The torch extension _fhog_torch against flash_hog/_hip.py's Python wrappers.

Both call the same C-ABI entry points; the extension does the checks,
allocations and the call in C++. On the same inputs their outputs must be
bitwise equal, their errors the same (type and message), and the extension
must enqueue on torch's current stream like the wrappers do.
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
