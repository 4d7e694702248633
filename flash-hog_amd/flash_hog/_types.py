"""Mask types of the attention front-ends.

The reference takes its MaskType from jax._src.cudnn.fused_attention_stablehlo
(flash_hog/jax/attention.py:10, :38); this enum keeps the members the
reference uses with the same names and values, without the JAX dependency.

CAUSAL is aligned top-left (key j visible to query i iff j <= i), the mask of
the reference's kernel (flash_hog/jax/_pallas_gpu_kernel.py:37-41) and of
cuDNN. CAUSAL_BOTTOM_RIGHT (key j visible iff j <= i + n_k - n_q) is the mask
of the reference's jax_refs (flash_hog/_jax_refs/jax_impl.py:104-109); it is
an addition of this package, valued outside the range of JAX's members.
"""

import dataclasses
import enum

# Values of the C ABI's `causal` argument (include/flash_hog.h, enum fhog_causal).
CAUSAL_NONE = 0
CAUSAL_TOP_LEFT = 1
CAUSAL_BOTTOM_RIGHT = 2


class MaskType(enum.IntEnum):
    NO_MASK = 0
    PADDING = 1
    CAUSAL = 2
    PADDING_CAUSAL = 3
    ALIBI = 4
    CAUSAL_BOTTOM_RIGHT = 16


_CODES = {
    MaskType.NO_MASK: CAUSAL_NONE,
    MaskType.CAUSAL: CAUSAL_TOP_LEFT,
    MaskType.CAUSAL_BOTTOM_RIGHT: CAUSAL_BOTTOM_RIGHT,
}


def causal_code(mask_type: MaskType) -> int:
    """The C ABI's causal code of a mask type; raises for the mask types the
    kernels do not implement (the reference allows NO_MASK and CAUSAL only,
    _pallas_gpu_kernel.py:100)."""
    mask_type = MaskType(mask_type)
    if mask_type not in _CODES:
        raise ValueError(f"only NO_MASK, CAUSAL and CAUSAL_BOTTOM_RIGHT are supported, got {mask_type.name}")
    return _CODES[mask_type]


def is_causal(mask_type: MaskType) -> bool:
    """True for the causal mask types (either alignment)."""
    return causal_code(mask_type) != CAUSAL_NONE


@dataclasses.dataclass(frozen=True)
class TuningConfig:
    """The reference's tile configuration of its Pallas kernel (same fields
    and defaults, flash_hog/jax/_pallas_gpu_kernel.py:22-29), accepted by
    flash_bwdbwd so that calls written for the reference run unchanged.

    The HIP kernels' tiles are compile-time constants chosen per dtype and
    head dim on MI355X (128 rows per workgroup, 32-row streamed tiles, 16 or
    32 rows per wave), and any sequence length works, so a TuningConfig does
    not change the kernels or their results; in the reference too it only
    changes speed (and requires sequence lengths divisible by its tiles,
    :84-86, which these kernels do not)."""
    tile_q: int
    tile_k: int
    max_concurrent_steps: int
    epilogue_tile_n: int = 64
    grid_minor_dim: int = 0
    grid_tile_width: int = 1
