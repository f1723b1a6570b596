"""MI355X-native drop-in for the `flash_attention_sm75` package.

Public surface identical to reference src/flash_attention_sm75/__init__.py:1-4.
"""
from .ops import (flash_attention, flash_attention_backward, flash_attention_forward,
                  flash_attention_forward_ex, flash_attention_forward_lse)

__version__ = "0.1.0"
__all__ = ["flash_attention_forward", "flash_attention_forward_ex", "flash_attention_forward_lse",
           "flash_attention", "flash_attention_backward"]
