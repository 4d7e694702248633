"""Attention with memory-linear second-order gradients, as torch autograd Functions.

Public entry point and rule structure of flash_hog/jax/attention.py:19-130:

  dot_product_attention(query, key, value, is_causal=False, scale=None)
    -> _DotProductAttention         (attention.py:52-60, custom_vjp #1)
         forward  = fwd rule         (attention.py:64-72)
         backward = _DotProductAttentionBwd.apply
    -> _DotProductAttentionBwd      (attention.py:100-107, custom_vjp #2)
         forward  = bwd_fwd rule     (attention.py:110-116)
         backward = bwd_bwd rule     (attention.py:119-125)

so torch.autograd.grad(..., create_graph=True) followed by a second grad
(grad-of-grad, Hessian-vector products) runs the HIP forward, first backward and
Flash-HOG double backward, never an (N_Q, N_K) tensor. As in the reference, the
double-backward rule returns no cotangent for the residuals L and O: the
rules compute total derivatives of (dQ, dK, dV) with respect to (q, k, v, dO).

The rules are looked up as module attributes of _attention_impl at call time
(attention.py:60, :70, :106, :115, :124), so they can be swapped at run time.

Eager calls with the default rules, outside torch.func transforms and compiler
traces, on plain GPU tensors, take the same two Functions written in C++
(flash-hog_amd/csrc/fhog_torch.cpp, AttentionFn and AttentionBwdFn): the
autograd engine then calls the kernels with no Python in between, which is
what bounds a Hessian-vector product at short sequences. Their results are
those of the Python Functions, bit for bit.
"""

from __future__ import annotations

import torch
from torch.autograd.function import once_differentiable

from flash_hog import _hip
from flash_hog._types import MaskType, causal_code
from flash_hog.torch import _attention_impl as attn_impl

# The rule bodies the C++ Functions reproduce; another one swapped in (a module
# attribute of _attention_impl) sends calls through the Python Functions.
_DEFAULT_RULES = (attn_impl.dot_product_attention_fwd_rule, attn_impl.dot_product_attention_bwd_rule,
                  attn_impl.dot_product_attention_bwd_rule_fwd_rule, attn_impl.dot_product_attention_bwd_rule_bwd_rule)


def _native_path(*tensors):
    """The torch extension whose attention() serves this call with C++
    autograd Functions, or None when the Python Functions must."""
    if (torch._C._are_functorch_transforms_active() or torch.compiler.is_compiling()
            or not all(type(t) is torch.Tensor and t.is_cuda for t in tensors)
            or attn_impl.dot_product_attention_fwd_rule is not _DEFAULT_RULES[0]
            or attn_impl.dot_product_attention_bwd_rule is not _DEFAULT_RULES[1]
            or attn_impl.dot_product_attention_bwd_rule_fwd_rule is not _DEFAULT_RULES[2]
            or attn_impl.dot_product_attention_bwd_rule_bwd_rule is not _DEFAULT_RULES[3]):
        return None
    return _hip.torch_ext()


# Head dims the kernels take, per dtype. Another head dim up to the largest is
# served by zero-padding q, k and v to the next one: padded columns add nothing
# to any score, give zero output columns, and their gradients are dropped by the
# padding's own backward, so the results are those of the unpadded problem (at
# the cost of the copies and of the padded columns' arithmetic).
_KERNEL_HEAD_DIMS = {torch.bfloat16: (64, 128, 256), torch.float16: (64, 128, 256), torch.float32: (64, 128)}


def kernel_head_dim(dtype, head_dim: int) -> int | None:
    """The head dim the kernels compute a problem of this head dim in (itself or
    the padded one), or None if none takes it."""
    for d in _KERNEL_HEAD_DIMS.get(dtype, ()):
        if head_dim <= d:
            return d
    return None


def dot_product_attention(query, key, value, is_causal: bool = False, scale: float | None = None, *,
                          causal_alignment: str = "top_left"):
    """Softmax attention over (B, T, N, H) or unbatched (T, N, H) tensors.

    Dimensions: T query length, S key/value length, N heads, H head dim
    (flash_hog/jax/attention.py:26-33). scale defaults to H ** -0.5. key and
    value may have fewer heads than query (a divisor: grouped-query attention,
    query head n uses key/value head n // (N / N_kv)).

    causal_alignment (an addition to the reference's signature) places the
    causal diagonal: "top_left" (key s visible to query t iff s <= t, the
    reference kernel's mask) or "bottom_right" (s <= t + S - T, the mask of
    flash_hog/_jax_refs/jax_impl.py:104-109); they agree when T == S.

    Like the reference's kernel, any head dim H >= 1 works up to the largest
    one the kernels take (256 for bf16 and fp16, 128 for fp32); head dims the
    kernels do not take natively (other than 64, 128, 256) are zero-padded to
    the next one they do.
    """
    if scale is None:
        scale = query.shape[-1] ** -0.5
    head_dim = query.shape[-1]
    padded = kernel_head_dim(query.dtype, head_dim)
    if padded is not None and padded != head_dim and key.shape[-1] == value.shape[-1] == head_dim:
        pad = lambda t: torch.nn.functional.pad(t, (0, padded - head_dim))
        out = dot_product_attention(pad(query), pad(key), pad(value), is_causal, scale,
                                    causal_alignment=causal_alignment)
        return out[..., :head_dim]
    dtype = query.dtype
    if not (dtype == key.dtype == value.dtype):
        raise ValueError(f"query, key and value must share a dtype, got {query.dtype}, {key.dtype}, {value.dtype}")
    if causal_alignment not in ("top_left", "bottom_right"):
        raise ValueError(f"causal_alignment must be 'top_left' or 'bottom_right', got {causal_alignment!r}")
    if not is_causal:
        mask_type = MaskType.NO_MASK
    elif causal_alignment == "top_left":
        mask_type = MaskType.CAUSAL
    else:
        mask_type = MaskType.CAUSAL_BOTTOM_RIGHT
    unbatched = query.ndim == 3
    if unbatched:
        query, key, value = query.unsqueeze(0), key.unsqueeze(0), value.unsqueeze(0)
    native = _native_path(query, key, value)
    if native is not None:
        result = native.attention(query, key, value, causal_code(mask_type), float(scale))
    else:
        fn = _DotProductAttention if torch._C._are_functorch_transforms_active() else _DotProductAttentionEager
        result, _ = fn.apply(query, key, value, mask_type, float(scale))
    if unbatched:
        result = result.squeeze(0)
    return result


# Both Functions keep their residuals among their inputs and outputs and save
# them in setup_context, so torch.func transforms (vmap, grad, jacrev) compose
# with them; under vmap the kernels' own vmap rules fold the mapped axis into
# the batch axis (flash_hog/torch/_hip_gpu.py).

class _DotProductAttention(torch.autograd.Function):
    """Primal: (q, k, v) -> (O, L); L = activation, the fwd rule's residual
    (attention.py:64-72), is returned so that it can be saved, and is not
    differentiable."""

    generate_vmap_rule = True

    @staticmethod
    def forward(query, key, value, mask_type, scale):
        out, (_, _, _, activation, _) = attn_impl.dot_product_attention_fwd_rule(
            query, key, value, mask_type=mask_type, scale=scale)
        return out, activation

    @staticmethod
    def setup_context(ctx, inputs, output):
        query, key, value, mask_type, scale = inputs
        out, activation = output
        # the residual (q, k, v, L, O) of dot_product_attention_fwd_rule
        ctx.save_for_backward(query, key, value, activation, out)
        ctx.mark_non_differentiable(activation)
        ctx.mask_type = mask_type
        ctx.scale = scale

    @staticmethod
    def backward(ctx, g, _g_activation):
        q, k, v, activation, o = ctx.saved_tensors
        # O enters the first backward as a constant (the double-backward rule
        # returns no cotangent for it); detaching it keeps this node out of the
        # graph of a second derivative, which would otherwise call it again with
        # a zero cotangent.
        fn = _DotProductAttentionBwd if torch._C._are_functorch_transforms_active() else _DotProductAttentionBwdEager
        dq, dk, dv = fn.apply(ctx.mask_type, ctx.scale, q, k, v, activation, o.detach(), g)
        return dq, dk, dv, None, None


class _DotProductAttentionBwd(torch.autograd.Function):
    """Primal: (q, k, v, L, O, dO) -> (dQ, dK, dV); differentiable in q, k, v, dO."""

    generate_vmap_rule = True

    @staticmethod
    def forward(mask_type, scale, query, key, value, activation, out, g):
        (dq, dk, dv), _ = attn_impl.dot_product_attention_bwd_rule_fwd_rule(
            mask_type=mask_type, scale=scale, res=(query, key, value, activation, out), g=g)
        return dq, dk, dv

    @staticmethod
    def setup_context(ctx, inputs, output):
        mask_type, scale, query, key, value, activation, out, g = inputs
        # the residual (q, k, v, O, L, dO) of dot_product_attention_bwd_rule_fwd_rule
        ctx.save_for_backward(query, key, value, out, activation, g)
        ctx.mask_type = mask_type
        ctx.scale = scale

    @staticmethod
    @once_differentiable
    def backward(ctx, ddq, ddk, ddv):
        # The rules stop at second order (as the reference's do): the outputs
        # of this backward raise if differentiated again.
        res = ctx.saved_tensors
        (dq2, dk2, dv2, _, _), ddo = attn_impl.dot_product_attention_bwd_rule_bwd_rule(
            mask_type=ctx.mask_type, scale=ctx.scale, res=res, g=(ddq, ddk, ddv))
        return None, None, dq2, dk2, dv2, None, None, ddo


# The same two Functions in the ctx-first form. Function.apply binds a
# setup_context-style Function's arguments through inspect.signature on every
# call (tens of microseconds of host time, twice per Hessian-vector product);
# the ctx-first form skips that. It cannot run under torch.func transforms, so
# the callers above pick it only when none is active.

class _DotProductAttentionEager(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, key, value, mask_type, scale):
        output = _DotProductAttention.forward(query, key, value, mask_type, scale)
        _DotProductAttention.setup_context(ctx, (query, key, value, mask_type, scale), output)
        return output

    backward = _DotProductAttention.backward


class _DotProductAttentionBwdEager(torch.autograd.Function):
    @staticmethod
    def forward(ctx, mask_type, scale, query, key, value, activation, out, g):
        output = _DotProductAttentionBwd.forward(mask_type, scale, query, key, value, activation, out, g)
        _DotProductAttentionBwd.setup_context(ctx, (mask_type, scale, query, key, value, activation, out, g), output)
        return output

    backward = _DotProductAttentionBwd.backward
