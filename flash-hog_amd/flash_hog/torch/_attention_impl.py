"""Rule bodies of the attention front-end, one function per reference rule.

Each function keeps the name, arguments and return structure of its
counterpart in flash_hog/jax/_attention_impl.py, with the cuDNN and Pallas
calls replaced by the HIP kernels of this package:

  dot_product_attention_fwd              :224-229  (cuDNN forward, no residual)
  dot_product_attention_fwd_rule         :232-239  (cuDNN forward + residual)
  dot_product_attention_bwd_rule         :242-261  (cuDNN backward)
  dot_product_attention_bwd_rule_fwd_rule:264-275  (backward saving (q,k,v,O,L,dO))
  dot_product_attention_bwd_rule_bwd_rule:278-303  (Flash-HOG double backward,
                                                    zero cotangents for L and O)

The reference's 12-tuple cuDNN residual (:200-221) only exists to satisfy
cuDNN's rule signature; here the residual is the 5-tuple (q, k, v, L, O) the
public rules pass around (flash_hog/jax/attention.py:71).
"""

from __future__ import annotations

from flash_hog._types import MaskType, TuningConfig
from flash_hog.torch import _hip_gpu


# The configuration the reference's rule passes (_attention_impl.py:297).
_CONFIG = TuningConfig(tile_q=32, tile_k=32, max_concurrent_steps=4)


def dot_product_attention_fwd(query, key, value, mask_type: MaskType, scale: float):
    out, _ = _hip_gpu.flash_fwd(query, key, value, mask_type=mask_type, scale=scale)
    return out


def dot_product_attention_fwd_rule(query, key, value, mask_type: MaskType, scale: float):
    out, activation = _hip_gpu.flash_fwd(query, key, value, mask_type=mask_type, scale=scale)
    res = (query, key, value, activation, out)
    return out, res


def dot_product_attention_bwd_rule(mask_type: MaskType, scale: float, res, g):
    query, key, value, activation, out = res
    return _hip_gpu.flash_bwd(query, key, value, out, g, activation, mask_type=mask_type, scale=scale)


def dot_product_attention_bwd_rule_fwd_rule(mask_type: MaskType, scale: float, res, g):
    query, key, value, activation, out = res
    dO = g
    dQ, dK, dV = dot_product_attention_bwd_rule(mask_type=mask_type, scale=scale, res=res, g=dO)
    residual = (query, key, value, out, activation, dO)
    return (dQ, dK, dV), residual


def dot_product_attention_bwd_rule_bwd_rule(mask_type: MaskType, scale: float, res, g):
    query, key, value, out, activation, dO = res
    ddQ, ddK, ddV = g
    dQ2, dK2, dV2, ddO = _hip_gpu.flash_bwdbwd(
        Q=query, K=key, V=value, O=out, dO=dO, ddQ=ddQ, ddK=ddK, ddV=ddV, L=activation,
        mask_type=mask_type, scale=scale, config=_CONFIG)
    d_res = (dQ2, dK2, dV2, None, None)
    return d_res, ddO
