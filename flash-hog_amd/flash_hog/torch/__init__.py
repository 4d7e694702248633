"""PyTorch front-end: flash_hog.torch.attention.dot_product_attention."""

from flash_hog.torch.attention import dot_product_attention

__all__ = ["dot_product_attention"]
