"""Mask types of the attention front-ends.

The reference takes its MaskType from jax._src.cudnn.fused_attention_stablehlo
(flash_hog/jax/attention.py:10, :38); this enum keeps the members the
reference uses with the same names and values, without the JAX dependency.
"""

import enum


class MaskType(enum.IntEnum):
    NO_MASK = 0
    PADDING = 1
    CAUSAL = 2
    PADDING_CAUSAL = 3
    ALIBI = 4


def is_causal(mask_type: MaskType) -> bool:
    """True for CAUSAL; raises for the mask types the kernels do not implement
    (the reference allows NO_MASK and CAUSAL only, _pallas_gpu_kernel.py:100)."""
    mask_type = MaskType(mask_type)
    if mask_type not in (MaskType.NO_MASK, MaskType.CAUSAL):
        raise ValueError(f"only NO_MASK and CAUSAL are supported, got {mask_type.name}")
    return mask_type == MaskType.CAUSAL
