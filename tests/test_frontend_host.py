"""Host logic of the torch front-end, without a GPU.

The kernel operators have fake (meta) implementations, so shape handling,
the vmap fold of the mapped axis into the batch axis (the reference's
custom_vmap rule, flash_hog/jax/_pallas_gpu.py:85-102), the composition of
the autograd rules with torch.func transforms, and argument validation run
here on meta tensors; no kernel is launched and no numerics are checked (the
GPU tests in test_gpu_frontend.py do that).
"""

from __future__ import annotations

import pytest
import torch

import flash_hog
from flash_hog._types import MaskType, causal_code, is_causal


def meta(*shape, dtype=torch.bfloat16):
    return torch.empty(*shape, device="meta", dtype=dtype)


def attn(q, k, v, **kw):
    return flash_hog.dot_product_attention(q, k, v, is_causal=True, **kw)


def test_mask_codes():
    assert causal_code(MaskType.NO_MASK) == 0
    assert causal_code(MaskType.CAUSAL) == 1
    assert causal_code(MaskType.CAUSAL_BOTTOM_RIGHT) == 2
    assert is_causal(MaskType.CAUSAL_BOTTOM_RIGHT) and not is_causal(MaskType.NO_MASK)
    with pytest.raises(ValueError, match="supported"):
        causal_code(MaskType.PADDING)


def test_alignment_is_validated():
    q = meta(1, 8, 2, 64)
    with pytest.raises(ValueError, match="causal_alignment"):
        flash_hog.dot_product_attention(q, q, q, is_causal=True, causal_alignment="diagonal")


def test_vmap_folds_the_mapped_axis():
    q, k, v = meta(3, 2, 64, 4, 64), meta(3, 2, 80, 2, 64), meta(3, 2, 80, 2, 64)
    out = torch.func.vmap(attn)(q, k, v)
    assert out.shape == q.shape
    out = torch.func.vmap(attn, in_dims=(0, None, None))(q, k[0], v[0])
    assert out.shape == q.shape
    out = torch.func.vmap(attn, in_dims=(2, 2, 2))(q.movedim(0, 2), k.movedim(0, 2), v.movedim(0, 2))
    assert out.shape == q.shape


def test_vmap_of_grad_and_of_hvp():
    q, k, v = meta(3, 2, 64, 4, 64), meta(3, 2, 80, 2, 64), meta(3, 2, 80, 2, 64)

    def loss(q, k, v):
        return attn(q, k, v, causal_alignment="bottom_right").float().sum()

    g = torch.func.vmap(torch.func.grad(loss, argnums=(0, 1, 2)))(q, k, v)
    assert [t.shape for t in g] == [q.shape, k.shape, v.shape]

    def g_dot_u(q, k, v, uq, uk, uv):
        gr = torch.func.grad(loss, argnums=(0, 1, 2))(q, k, v)
        return sum((a.float() * b.float()).sum() for a, b in zip(gr, (uq, uk, uv)))

    h = torch.func.vmap(torch.func.grad(g_dot_u, argnums=(0, 1, 2)))(q, k, v, q, k, v)
    assert [t.shape for t in h] == [q.shape, k.shape, v.shape]


def test_grad_of_grad_stops_at_second_order():
    q = meta(2, 16, 4, 64).requires_grad_(True)
    k = meta(2, 16, 2, 64).requires_grad_(True)
    v = meta(2, 16, 2, 64).requires_grad_(True)
    out = attn(q, k, v)
    g = torch.autograd.grad(out, (q, k, v), torch.empty_like(out), create_graph=True)
    assert all(t.requires_grad for t in g)
    h = torch.autograd.grad(g, (q, k, v), tuple(torch.empty_like(t) for t in g), create_graph=True)
    assert [t.shape for t in h] == [q.shape, k.shape, v.shape]
    assert not any(t.requires_grad for t in h)


def test_native_path_only_for_plain_gpu_tensors():
    """The C++ autograd Functions serve plain GPU tensors only: meta and CPU
    tensors (and tensor subclasses) go through the Python Functions, whose
    operators have the fake kernels used above."""
    from flash_hog.torch import attention as att

    assert att._native_path(meta(1, 8, 2, 64)) is None
    assert att._native_path(torch.zeros(1, 8, 2, 64)) is None

    class Sub(torch.Tensor):
        pass

    assert att._native_path(torch.zeros(1, 8, 2, 64).as_subclass(Sub)) is None


def test_unbatched_shapes():
    q, k = meta(64, 4, 64), meta(80, 2, 64)
    assert attn(q, k, k).shape == q.shape


def test_padded_head_dims_keep_shapes():
    """Head dims the kernels do not take natively are zero-padded to 64, 128 or 256
    and sliced back; the derivatives keep the caller's shapes."""
    from flash_hog.torch.attention import kernel_head_dim

    assert kernel_head_dim(torch.bfloat16, 96) == 128 and kernel_head_dim(torch.bfloat16, 1) == 64
    assert kernel_head_dim(torch.float16, 128) == 128 and kernel_head_dim(torch.bfloat16, 129) == 256
    assert kernel_head_dim(torch.bfloat16, 257) is None and kernel_head_dim(torch.float16, 200) == 256
    assert kernel_head_dim(torch.float32, 48) == 64 and kernel_head_dim(torch.float32, 96) == 128
    assert kernel_head_dim(torch.float32, 129) is None
    q = meta(2, 16, 4, 96).requires_grad_(True)
    k = meta(2, 16, 2, 96).requires_grad_(True)
    v = meta(2, 16, 2, 96).requires_grad_(True)
    out = attn(q, k, v)
    assert out.shape == q.shape
    g = torch.autograd.grad(out, (q, k, v), torch.empty_like(out), create_graph=True)
    h = torch.autograd.grad(g, (q, k, v), tuple(torch.empty_like(t) for t in g))
    assert [t.shape for t in h] == [q.shape, k.shape, v.shape]
    out = torch.func.vmap(attn)(meta(3, 2, 16, 4, 40), meta(3, 2, 16, 4, 40), meta(3, 2, 16, 4, 40))
    assert out.shape == (3, 2, 16, 4, 40)


def test_torch_compile_traces_forward_and_gradient():
    """torch.compile (aot_eager backend, whole graph, no graph break) traces
    the forward and its gradient through the kernel operators' fake
    implementations. A second derivative of a compiled graph is refused by
    torch itself (aot_autograd graphs are once differentiable); eager
    grad-of-grad is what the GPU tests cover."""
    q, k, v = meta(2, 64, 4, 64), meta(2, 64, 2, 64), meta(2, 64, 2, 64)
    out = torch.compile(attn, backend="aot_eager", fullgraph=True)(q, k, v)
    assert out.shape == q.shape

    def loss(q, k, v):
        return attn(q, k, v, causal_alignment="bottom_right").float().sum()

    qr, kr, vr = (t.clone().requires_grad_(True) for t in (q, k, v))
    g = torch.autograd.grad(torch.compile(loss, backend="aot_eager", fullgraph=True)(qr, kr, vr), (qr, kr, vr))
    assert [t.shape for t in g] == [q.shape, k.shape, v.shape]


def test_flash_bwdbwd_takes_the_reference_tuning_config():
    """flash_bwdbwd accepts the reference's TuningConfig (same fields and
    defaults, _pallas_gpu_kernel.py:22-29) and rejects anything else as config."""
    from flash_hog import TuningConfig
    from flash_hog.torch import _hip_gpu

    cfg = TuningConfig(tile_q=32, tile_k=32, max_concurrent_steps=4)
    assert (cfg.epilogue_tile_n, cfg.grid_minor_dim, cfg.grid_tile_width) == (64, 0, 1)
    q, k = meta(1, 64, 2, 64), meta(1, 64, 2, 64)
    lse = meta(1, 2, 64, dtype=torch.float32)
    outs = _hip_gpu.flash_bwdbwd(q, k, k, q, q, q, k, k, lse, mask_type=MaskType.CAUSAL, scale=None, config=cfg)
    assert [t.shape for t in outs] == [q.shape, k.shape, k.shape, q.shape]
    with pytest.raises(TypeError, match="TuningConfig"):
        _hip_gpu.flash_bwdbwd(q, k, k, q, q, q, k, k, lse, mask_type=MaskType.CAUSAL, scale=None, config={"tile_q": 32})
