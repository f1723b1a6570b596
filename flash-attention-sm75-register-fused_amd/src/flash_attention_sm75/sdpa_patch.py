"""Monkey-patch of ``torch.nn.functional.scaled_dot_product_attention``.

Mirrors reference examples/llama_attention_replacement.py:18-119: the same
names (``apply_patch``, ``remove_patch``, ``patch_stats``, ``_stats``,
``_patched_sdpa``, ``_original_sdpa``), the same statistics layout and the same
fallback reasons, so HuggingFace models that call SDPA (transformers'
``sdpa_attention_forward`` looks the function up on every call) run their
attention through the gfx950 kernel.

Differences from the reference, all of which widen what runs on the kernel
without changing results:
  * calls with ``N_q != N_k`` (KV-cache decode, chunked prefill) use the
    kernel instead of falling back; ``is_causal`` keeps SDPA's top-left
    alignment (key j visible to query i iff j <= i);
  * boolean ``attn_mask`` (what transformers builds for padded batches) runs
    on the kernel too; additive float masks fall back, and so does a mask
    given together with ``is_causal`` (reason ``mask_and_causal``): torch
    documents that pair as an error, and its behaviour differs between
    devices and builds, so the call goes to torch unchanged and raises (or
    returns) exactly what the unpatched call does;
  * Q/K/V views are read in place (transformers passes [B, N, H, D] buffers
    viewed as [B, H, N, D]) and O keeps Q's layout, so the caller's
    ``transpose(1, 2).contiguous()`` is free;
  * grouped K/V heads go to the kernel as they are (no repeat_interleave)
    when the call says ``enable_gqa=True``; without it torch's SDPA rejects
    grouped heads, so such calls pass through to torch and raise there;
  * bfloat16 calls (most current models' dtype) run on the kernel's bfloat16
    instances; other dtypes, and mixed ones, fall back;
  * calls that need gradients (training) run on :func:`flash_attention`,
    whose backward is the fused dQ/dK/dV kernels (boolean masks included).
"""
import torch
import torch.nn.functional as F

from .ops import flash_attention, flash_attention_forward_ex

_original_sdpa = F.scaled_dot_product_attention
_patch_active = False

_stats = {
    "total": 0,
    "flash": 0,
    "fallback": 0,
    "fallback_reasons": {},
}


def _record_fallback(reason: str):
    _stats["fallback"] += 1
    _stats["fallback_reasons"][reason] = _stats["fallback_reasons"].get(reason, 0) + 1


def _fallback_reason(query, key, value, attn_mask, dropout_p, is_causal, kwargs):
    """Why a call cannot run on the kernel, or None (reference :47-64)."""
    if not query.is_cuda:
        return "not_cuda"
    if (query.dtype not in (torch.float16, torch.bfloat16) or key.dtype != query.dtype
            or value.dtype != query.dtype):
        return "not_fp16"  # the reference's name; bfloat16 runs on the kernel too
    if query.dim() != 4 or key.dim() != 4 or value.dim() != 4:
        return "not_4d"
    if query.size(-1) not in (64, 128):
        return "head_dim_unsupported"
    if key.size(-1) != query.size(-1) or value.shape != key.shape:
        return "kv_shape_mismatch"
    if dropout_p != 0.0:
        return "dropout"
    if attn_mask is not None and attn_mask.dtype != torch.bool:
        return "has_attn_mask"  # additive float masks stay with torch
    if attn_mask is not None and is_causal:
        return "mask_and_causal"  # torch's own call decides (it documents an error)
    if key.size(0) != query.size(0):
        return "batch_mismatch"
    if key.size(1) == 0 or query.size(1) % key.size(1) != 0:
        return "heads_not_divisible"
    if query.size(1) != key.size(1) and not kwargs.get("enable_gqa", False):
        return "gqa_not_enabled"  # torch raises for grouped heads without enable_gqa
    if key.size(2) == 0:
        return "empty_kv"
    if set(kwargs) - {"enable_gqa"}:
        return "unsupported_kwargs"
    return None


def _needs_grad(query, key, value):
    return torch.is_grad_enabled() and (query.requires_grad or key.requires_grad
                                        or value.requires_grad)


def _patched_sdpa(query, key, value, attn_mask=None, dropout_p=0.0, is_causal=False,
                  scale=None, **kwargs):
    _stats["total"] += 1
    reason = _fallback_reason(query, key, value, attn_mask, dropout_p, is_causal, kwargs)
    if reason is not None:
        _record_fallback(reason)
        # everything passes through unchanged
        return _original_sdpa(query, key, value, attn_mask=attn_mask, dropout_p=dropout_p,
                              is_causal=is_causal, scale=scale, **kwargs)
    _stats["flash"] += 1
    if _needs_grad(query, key, value):
        return flash_attention(query, key, value, causal=bool(is_causal), scale=scale,
                               attn_mask=attn_mask)
    return flash_attention_forward_ex(query, key, value, causal=bool(is_causal), scale=scale,
                                      attn_mask=attn_mask)


def apply_patch():
    global _patch_active
    if _patch_active:
        return
    F.scaled_dot_product_attention = _patched_sdpa
    torch.nn.functional.scaled_dot_product_attention = _patched_sdpa
    _patch_active = True
    print("[flash-attention-sm75] Patch applied.")


def remove_patch():
    global _patch_active
    F.scaled_dot_product_attention = _original_sdpa
    torch.nn.functional.scaled_dot_product_attention = _original_sdpa
    _patch_active = False
    print("[flash-attention-sm75] Patch removed.")


def patch_stats():
    return dict(_stats, active=_patch_active)


def reset_stats():
    _stats["total"] = 0
    _stats["flash"] = 0
    _stats["fallback"] = 0
    _stats["fallback_reasons"].clear()
