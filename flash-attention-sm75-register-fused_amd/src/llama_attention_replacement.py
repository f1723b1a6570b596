"""Import-compatible stand-in for reference examples/llama_attention_replacement.py.

The reference's prefill test imports ``apply_patch, remove_patch, _stats``
from a module of this name (reference tests/test_prefill_correctness.py:
11-12); the implementation lives in ``flash_attention_sm75.sdpa_patch``.
"""
from flash_attention_sm75.sdpa_patch import (  # noqa: F401
    _original_sdpa,
    _patched_sdpa,
    _record_fallback,
    _stats,
    apply_patch,
    patch_stats,
    remove_patch,
    reset_stats,
)
