"""Dispatch layer between the rule bodies and the HIP kernels.

flash_bwdbwd mirrors flash_hog/jax/_pallas_gpu.py:51-114: unbatched (T, N, H)
arguments get a leading batch axis, which is removed from the results, and the
kernel call itself goes through the C ABI (flash_hog/_hip.py). flash_fwd and
flash_bwd are the same wrappers around the forward and first backward, whose
reference counterparts are cuDNN calls (flash_hog/jax/_attention_impl.py:229,
:248). The default scale is head_dim ** -0.5 (_pallas_gpu_kernel.py:103-104).
"""

from __future__ import annotations

from flash_hog import _hip
from flash_hog._types import MaskType, is_causal


def _default_scale(x, scale):
    return x.shape[-1] ** -0.5 if scale is None else float(scale)


def _batchify(*xs):
    return tuple(None if x is None else x.unsqueeze(0) for x in xs)


def flash_fwd(query, key, value, *, mask_type: MaskType, scale: float | None):
    """Returns (out, activation): out like query, activation = L (B, N, T) fp32."""
    if query.ndim == 3:
        out, lse = flash_fwd(*_batchify(query, key, value), mask_type=mask_type, scale=scale)
        return out[0], lse[0]
    return _hip.attention_fwd(query, key, value, is_causal(mask_type), _default_scale(query, scale))


def flash_bwd(query, key, value, out, dO, activation, *, mask_type: MaskType, scale: float | None):
    """Returns (dQ, dK, dV)."""
    if query.ndim == 3:
        res = flash_bwd(*_batchify(query, key, value, out, dO, activation), mask_type=mask_type, scale=scale)
        return tuple(r[0] for r in res)
    dq, dk, dv, _ = _hip.attention_bwd(query, key, value, out, dO, activation,
                                       is_causal(mask_type), _default_scale(query, scale))
    return dq, dk, dv


def flash_bwdbwd(Q, K, V, O, dO, ddQ, ddK, ddV, L, *, mask_type: MaskType, scale: float | None):
    """Returns (dQ2, dK2, dV2, ddO) (flash_hog/jax/_pallas_gpu.py:51-114)."""
    if Q.ndim == 3:
        res = flash_bwdbwd(*_batchify(Q, K, V, O, dO, ddQ, ddK, ddV, L), mask_type=mask_type, scale=scale)
        return tuple(r[0] for r in res)
    return _hip.attention_bwdbwd(Q, K, V, O, dO, ddQ, ddK, ddV, L,
                                 is_causal(mask_type), _default_scale(Q, scale))
