"""MI355X-native Flash-HOG: attention with memory-linear second-order gradients.

The reference re-exports its JAX entry point here (flash_hog/__init__.py:1).
JAX is not a dependency of this package, so the package root re-exports the
PyTorch front-end with the same signature; both call the same HIP kernels
through the C ABI in include/flash_hog.h.
"""

from flash_hog._types import MaskType, TuningConfig
from flash_hog.torch._hip_gpu import supported
from flash_hog.torch.attention import dot_product_attention

__all__ = ["MaskType", "TuningConfig", "dot_product_attention", "supported"]
