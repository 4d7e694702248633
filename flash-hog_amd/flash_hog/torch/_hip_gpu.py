"""Dispatch layer between the rule bodies and the HIP kernels.

flash_bwdbwd mirrors flash_hog/jax/_pallas_gpu.py:51-114: unbatched (T, N, H)
arguments get a leading batch axis, which is removed from the results, and the
kernel call goes through the C ABI (flash_hog/_hip.py). flash_fwd and
flash_bwd are the same wrappers around the forward and first backward, whose
reference counterparts are cuDNN calls (flash_hog/jax/_attention_impl.py:229,
:248). The default scale is head_dim ** -0.5 (_pallas_gpu_kernel.py:103-104).

Each kernel call is a torch custom operator (flash_hog::attention_fwd,
::attention_bwd, ::attention_bwdbwd) with a vmap rule that folds the mapped
axis into the batch axis, calls the kernel once and unfolds the results: the
reference's custom_vmap rule (_pallas_gpu.py:85-102, "(new_batch old_batch)"),
which lets torch.func.vmap map the front-end without a per-element loop.
Unlike the reference, which asserts that every argument is mapped (:88), an
unmapped argument is broadcast along the mapped axis. Fake (meta) kernels give
the output shapes to tracing tools.
"""

from __future__ import annotations

import torch

from flash_hog import _hip
from flash_hog._types import MaskType, TuningConfig, causal_code


def _default_scale(x, scale):
    return x.shape[-1] ** -0.5 if scale is None else float(scale)


def _batchify(*xs):
    return tuple(None if x is None else x.unsqueeze(0) for x in xs)


# --------------------------------------------------------------- operators

Tensor = torch.Tensor


@torch.library.custom_op("flash_hog::attention_fwd", mutates_args=())
def attention_fwd_op(q: Tensor, k: Tensor, v: Tensor, causal: int, scale: float) -> tuple[Tensor, Tensor]:
    return _hip.attention_fwd(q, k, v, causal, scale)


@torch.library.custom_op("flash_hog::attention_bwd", mutates_args=())
def attention_bwd_op(q: Tensor, k: Tensor, v: Tensor, o: Tensor, dout: Tensor, lse: Tensor, causal: int,
                     scale: float) -> tuple[Tensor, Tensor, Tensor]:
    dq, dk, dv, _ = _hip.attention_bwd(q, k, v, o, dout, lse, causal, scale)
    return dq, dk, dv


@torch.library.custom_op("flash_hog::attention_bwdbwd", mutates_args=())
def attention_bwdbwd_op(q: Tensor, k: Tensor, v: Tensor, o: Tensor, dout: Tensor, ddq: Tensor, ddk: Tensor,
                        ddv: Tensor, lse: Tensor, causal: int,
                        scale: float) -> tuple[Tensor, Tensor, Tensor, Tensor]:
    return _hip.attention_bwdbwd(q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale)


def _row_stats(q):
    B, T, N, _ = q.shape
    return q.new_empty((B, N, T), dtype=torch.float32)


@attention_fwd_op.register_fake
def _(q, k, v, causal, scale):
    return torch.empty_like(q), _row_stats(q)


@attention_bwd_op.register_fake
def _(q, k, v, o, dout, lse, causal, scale):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


@attention_bwdbwd_op.register_fake
def _(q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v), torch.empty_like(dout)


def _fold(info, in_dims, tensors):
    """Moves each mapped axis to the front (broadcasting unmapped tensors) and
    merges it with the batch axis: (V, B, ...) -> (V * B, ...)."""
    out = []
    for t, d in zip(tensors, in_dims):
        t = t.movedim(d, 0) if d is not None else t.unsqueeze(0).expand(info.batch_size, *t.shape)
        out.append(t.reshape(t.shape[0] * t.shape[1], *t.shape[2:]))
    return out


def _unfold(info, results):
    return tuple(r.unflatten(0, (info.batch_size, -1)) for r in results), (0,) * len(results)


@attention_fwd_op.register_vmap
def _(info, in_dims, q, k, v, causal, scale):
    return _unfold(info, attention_fwd_op(*_fold(info, in_dims[:3], (q, k, v)), causal, scale))


@attention_bwd_op.register_vmap
def _(info, in_dims, q, k, v, o, dout, lse, causal, scale):
    return _unfold(info, attention_bwd_op(*_fold(info, in_dims[:6], (q, k, v, o, dout, lse)), causal, scale))


@attention_bwdbwd_op.register_vmap
def _(info, in_dims, q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale):
    args = _fold(info, in_dims[:9], (q, k, v, o, dout, ddq, ddk, ddv, lse))
    return _unfold(info, attention_bwdbwd_op(*args, causal, scale))


# ------------------------------------------------------------ kernel calls
#
# The rules call the operators through these autograd Functions. A rule body
# may run inside a backward pass that is itself recorded (create_graph=True,
# nested torch.func.grad); the Function then stands for the kernel in that
# record, and asking for its derivative (a third-order derivative of
# attention) is an explicit error. setup_context and generate_vmap_rule make
# them usable under torch.func transforms, where vmap reaches the operators'
# own vmap rules.

def _no_derivative(name):
    def backward(ctx, *grads):
        raise NotImplementedError(
            f"{name} has no derivative of its own: differentiate through "
            "flash_hog.dot_product_attention, whose rules give the first and second derivatives")

    return staticmethod(backward)


def _mark_outputs(ctx, inputs, output):
    ctx.mark_non_differentiable(*output)


# forward spells out its parameters: torch.compile reads a forward whose first
# parameter is variadic as one that takes ctx.
class _FwdKernel(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(q, k, v, causal, scale):
        return attention_fwd_op(q, k, v, causal, scale)

    setup_context = staticmethod(_mark_outputs)
    backward = _no_derivative("flash_hog_attention_fwd")


class _BwdKernel(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(q, k, v, o, dout, lse, causal, scale):
        return attention_bwd_op(q, k, v, o, dout, lse, causal, scale)

    setup_context = staticmethod(_mark_outputs)
    backward = _no_derivative("flash_hog_attention_bwd")


class _BwdBwdKernel(torch.autograd.Function):
    generate_vmap_rule = True

    @staticmethod
    def forward(q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale):
        return attention_bwdbwd_op(q, k, v, o, dout, ddq, ddk, ddv, lse, causal, scale)

    setup_context = staticmethod(_mark_outputs)
    backward = _no_derivative("flash_hog_attention_bwdbwd")


# ---------------------------------------------------------------- wrappers
#
# Eager calls with gradient recording off (which is how the rules call them:
# inside an autograd Function's forward, or inside a once-differentiable
# backward) on plain GPU tensors, with no torch.func transform or compiler
# trace active, go straight to the C ABI: the Function and the operator would only
# add host time there (about 20 us per call), and their outputs would be the
# same tensors.

def _direct(*tensors) -> bool:
    return (not torch.is_grad_enabled() and not torch._C._are_functorch_transforms_active()
            and not torch.compiler.is_compiling() and tensors[0].is_cuda
            and all(type(t) is torch.Tensor for t in tensors))


def flash_fwd(query, key, value, *, mask_type: MaskType, scale: float | None):
    """Returns (out, activation): out like query, activation = L (B, N, T) fp32."""
    if query.ndim == 3:
        out, lse = flash_fwd(*_batchify(query, key, value), mask_type=mask_type, scale=scale)
        return out[0], lse[0]
    if _direct(query, key, value):
        return _hip.attention_fwd(query, key, value, causal_code(mask_type), _default_scale(query, scale))
    return _FwdKernel.apply(query, key, value, causal_code(mask_type), _default_scale(query, scale))


def flash_bwd(query, key, value, out, dO, activation, *, mask_type: MaskType, scale: float | None):
    """Returns (dQ, dK, dV)."""
    if query.ndim == 3:
        res = flash_bwd(*_batchify(query, key, value, out, dO, activation), mask_type=mask_type, scale=scale)
        return tuple(r[0] for r in res)
    if _direct(query, key, value, out, dO, activation):
        return _hip.attention_bwd(query, key, value, out, dO, activation, causal_code(mask_type),
                                  _default_scale(query, scale))[:3]
    return _BwdKernel.apply(query, key, value, out, dO, activation, causal_code(mask_type),
                            _default_scale(query, scale))


def flash_bwdbwd(Q, K, V, O, dO, ddQ, ddK, ddV, L, *, mask_type: MaskType, scale: float | None,
                 config: TuningConfig | None = None):
    """Returns (dQ2, dK2, dV2, ddO) (flash_hog/jax/_pallas_gpu.py:51-114).
    config is the reference's tile configuration, accepted and type-checked
    for call compatibility; the HIP kernels' tiles are fixed (TuningConfig)."""
    if config is not None and not isinstance(config, TuningConfig):
        raise TypeError(f"config must be a flash_hog TuningConfig, got {type(config).__name__}")
    if Q.ndim == 3:
        res = flash_bwdbwd(*_batchify(Q, K, V, O, dO, ddQ, ddK, ddV, L), mask_type=mask_type, scale=scale)
        return tuple(r[0] for r in res)
    if _direct(Q, K, V, O, dO, ddQ, ddK, ddV, L):
        return _hip.attention_bwdbwd(Q, K, V, O, dO, ddQ, ddK, ddV, L, causal_code(mask_type),
                                     _default_scale(Q, scale))
    return _BwdBwdKernel.apply(Q, K, V, O, dO, ddQ, ddK, ddV, L, causal_code(mask_type), _default_scale(Q, scale))


# ------------------------------------------------------------- capability

def supported(*, is_causal: bool, seq_len: int, head_dim: int, num_q_heads: int, num_kv_heads: int,
              dtype: torch.dtype = torch.bfloat16, kv_seq_len: int | None = None, batch: int = 1,
              scale: float | None = None, causal_alignment: str = "top_left",
              device: torch.device | int | None = None) -> bool:
    """True iff the HIP kernels can serve this problem on this machine: the
    library loads, the device (default: the current one) is a gfx950 GPU and
    the sizes, dtype, mask and scale are ones the kernels take. The keyword
    names and their meaning follow flash_hog/jax/_tk_gpu.py:70-80; kv_seq_len
    (default seq_len), batch, dtype, scale (default head_dim ** -0.5) and
    causal_alignment are the further arguments this library's limits depend on.
    Head dims that dot_product_attention zero-pads to one the kernels take
    count as supported. Nothing is launched or allocated."""
    if causal_alignment not in ("top_left", "bottom_right"):
        raise ValueError(f"causal_alignment must be 'top_left' or 'bottom_right', got {causal_alignment!r}")
    if head_dim < 1:
        return False  # no kernel takes it, and it has no default scale
    try:
        if device is None:
            if not torch.cuda.is_available():
                return False
            device = torch.cuda.current_device()
        index = device if isinstance(device, int) else torch.device(device).index
        if index is None:
            index = torch.cuda.current_device()
        mask = (MaskType.NO_MASK if not is_causal else
                MaskType.CAUSAL if causal_alignment == "top_left" else MaskType.CAUSAL_BOTTOM_RIGHT)
        from flash_hog.torch.attention import kernel_head_dim

        kernel_dim = kernel_head_dim(dtype, head_dim)
        ok, _ = _hip.attention_supported(batch, seq_len, seq_len if kv_seq_len is None else kv_seq_len, num_q_heads,
                                         num_kv_heads, head_dim if kernel_dim is None else kernel_dim, dtype,
                                         causal_code(mask), head_dim ** -0.5 if scale is None else scale,
                                         device=index)
        return ok
    except (ImportError, OSError):
        return False
