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
"""

from __future__ import annotations

import torch

from flash_hog._types import MaskType
from flash_hog.torch import _attention_impl as attn_impl


def dot_product_attention(query, key, value, is_causal: bool = False, scale: float | None = None):
    """Softmax attention over (B, T, N, H) or unbatched (T, N, H) tensors.

    Dimensions: T query length, S key/value length, N heads, H head dim
    (flash_hog/jax/attention.py:26-33). scale defaults to H ** -0.5.
    """
    if scale is None:
        scale = query.shape[-1] ** -0.5
    dtype = query.dtype
    if not (dtype == key.dtype == value.dtype):
        raise ValueError(f"query, key and value must share a dtype, got {query.dtype}, {key.dtype}, {value.dtype}")
    mask_type = MaskType.CAUSAL if is_causal else MaskType.NO_MASK
    unbatched = query.ndim == 3
    if unbatched:
        query, key, value = query.unsqueeze(0), key.unsqueeze(0), value.unsqueeze(0)
    result = _DotProductAttention.apply(query, key, value, mask_type, float(scale))
    if unbatched:
        result = result.squeeze(0)
    return result


class _DotProductAttention(torch.autograd.Function):
    @staticmethod
    def forward(ctx, query, key, value, mask_type, scale):
        out, res = attn_impl.dot_product_attention_fwd_rule(query, key, value, mask_type=mask_type, scale=scale)
        q, k, v, activation, o = res
        ctx.save_for_backward(q, k, v, activation, o.detach())
        ctx.mask_type = mask_type
        ctx.scale = scale
        return out

    @staticmethod
    def backward(ctx, g):
        q, k, v, activation, o = ctx.saved_tensors
        dq, dk, dv = _DotProductAttentionBwd.apply(ctx.mask_type, ctx.scale, q, k, v, activation, o, g)
        return dq, dk, dv, None, None


class _DotProductAttentionBwd(torch.autograd.Function):
    """Primal: (q, k, v, L, O, dO) -> (dQ, dK, dV); differentiable in q, k, v, dO."""

    @staticmethod
    def forward(ctx, mask_type, scale, query, key, value, activation, out, g):
        (dq, dk, dv), residual = attn_impl.dot_product_attention_bwd_rule_fwd_rule(
            mask_type=mask_type, scale=scale, res=(query, key, value, activation, out), g=g)
        ctx.save_for_backward(*residual)
        ctx.mask_type = mask_type
        ctx.scale = scale
        return dq, dk, dv

    @staticmethod
    def backward(ctx, ddq, ddk, ddv):
        res = ctx.saved_tensors
        (dq2, dk2, dv2, _, _), ddo = attn_impl.dot_product_attention_bwd_rule_bwd_rule(
            mask_type=ctx.mask_type, scale=ctx.scale, res=res, g=(ddq, ddk, ddv))
        return None, None, dq2, dk2, dv2, None, None, ddo
