"""Python API of the fused attention forward (gfx950).

Mirrors reference src/flash_attention_sm75/ops.py:1-82: same names, defaults,
argument meaning and error texts.  One behavioural difference, by design:
grouped-query attention no longer materialises ``repeat_interleave`` copies of
K and V (reference ops.py:24-26); the kernel maps query head ``h`` to KV head
``h // (Hq // Hkv)`` by index, which is the same mapping.

The native module ``flash_attn_sm75_cuda`` is required: importing this
package without it raises ImportError (there is no CPU fallback).
"""
import math

import torch

import flash_attn_sm75_cuda as _C


def _expand_kv_for_gqa(Q: torch.Tensor, K: torch.Tensor, V: torch.Tensor):
    """Explicit GQA/MQA expansion of K and V to Q's head count.

    Kept for callers of the reference helper (reference ops.py:6-27).  The
    forward path does not call it; it only checks divisibility with
    :func:`_check_gqa_heads`.
    """
    _check_gqa_heads(Q, K)
    h_q, h_kv = Q.size(1), K.size(1)
    if h_q == h_kv:
        return K, V
    factor = h_q // h_kv
    K = K.repeat_interleave(factor, dim=1).contiguous()
    V = V.repeat_interleave(factor, dim=1).contiguous()
    return K, V


def _check_gqa_heads(Q: torch.Tensor, K: torch.Tensor) -> None:
    h_q, h_kv = Q.size(1), K.size(1)
    if h_kv == 0 or h_q % h_kv != 0:
        raise RuntimeError(
            f"GQA expansion: Q heads ({h_q}) not divisible by K/V heads ({h_kv})"
        )


def _fused_forward(Q, K, V, causal, scale):
    _check_gqa_heads(Q, K)
    Q = Q.contiguous()
    K = K.contiguous()
    V = V.contiguous()
    return Q, K, V, _C.flash_attention_forward(Q, K, V, bool(causal), float(scale))


class FlashAttentionSM75Function(torch.autograd.Function):
    """Forward-only autograd function (reference ops.py:30-52)."""

    @staticmethod
    def forward(ctx, Q, K, V, causal, scale):
        Q, K, V, out = _fused_forward(Q, K, V, causal, scale)
        ctx.save_for_backward(Q, K, V, out)
        return out

    @staticmethod
    def backward(ctx, grad_output):
        raise NotImplementedError(
            "Backward pass is not implemented. "
            "flash-attention-sm75 is for inference only."
        )


def _check_inputs(Q):
    if Q.dim() != 4:
        raise ValueError("Q must be 4D [B, H, N, D]")
    head_dim = Q.size(-1)
    if head_dim not in (64, 128):
        raise RuntimeError(
            f"flash_attention_sm75 supports head_dim=64 or 128, got {head_dim}"
        )
    return head_dim


def flash_attention_forward(Q, K, V, causal=False, scale=None):
    """Fused attention forward, drop-in for reference ops.py:55-82.

    Args:
        Q: [B, H_q,  N, D]  float16, on the GPU
        K: [B, H_kv, N, D]  float16, H_kv divides H_q
        V: [B, H_kv, N, D]  float16
        causal: key j is visible to query i iff j <= i
        scale: softmax scale (default 1/sqrt(D))

    Returns:
        O: [B, H_q, N, D] float16
    """
    head_dim = _check_inputs(Q)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    if torch.is_grad_enabled() and (Q.requires_grad or K.requires_grad or V.requires_grad):
        return FlashAttentionSM75Function.apply(Q, K, V, causal, scale)
    # No graph is recorded for these inputs: the same forward without the
    # autograd Function's per-call cost (inference, e.g. under no_grad).
    return _fused_forward(Q, K, V, causal, scale)[3]


def flash_attention_forward_lse(Q, K, V, causal=False, scale=None):
    """Forward that also returns the fp32 row log-sum-exp.

    No reference counterpart (the reference lists LSE as future work).
    Returns ``(O, LSE)`` with LSE [B, H_q, N] float32, natural log of
    sum_j exp(scale * q_i . k_j) over the visible keys.
    """
    head_dim = _check_inputs(Q)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    _check_gqa_heads(Q, K)
    return _C.flash_attention_forward_lse(
        Q.contiguous(), K.contiguous(), V.contiguous(), bool(causal), float(scale)
    )


_CAUSAL_CODES = {False: 0, True: 1, "top_left": 1, "bottom_right": 2}


def flash_attention_forward_ex(Q, K, V, causal=False, scale=None, return_lse=False,
                               attn_mask=None):
    """Forward over separate query/key lengths and strided views.

    No reference counterpart: the reference binding requires Nq == Nk and
    contiguous tensors (reference pytorch_extension.cpp:22-25,61).

    Args:
        Q: [B, H_q, N_q, D] float16 or bfloat16 on the GPU; any layout whose
           head_dim is contiguous and whose other strides are multiples of 8
           is read in place (e.g. a [B, N, H, D] buffer viewed as
           [B, H, N, D]), other layouts are copied first.  With bfloat16 the
           probabilities are rounded to bfloat16 before the P V product.
        K, V: [B, H_kv, N_k, D], Q's dtype, H_kv divides H_q.
        causal: False; True or "top_left" (key j visible to query i iff
            j <= i, torch SDPA's is_causal); "bottom_right" (iff
            j <= i + N_k - N_q).  A query that sees no key gets a zero row.
        scale: softmax scale (default 1/sqrt(D)).
        return_lse: also return the fp32 natural-log row LSE [B, H_q, N_q].
        attn_mask: optional bool tensor broadcastable to [B, H_q, N_q, N_k],
            True = the key takes part (torch SDPA's boolean attn_mask); it is
            packed to bits on the GPU and combines with ``causal``.

    Returns:
        O [B, H_q, N_q, D] in Q's dtype with Q's memory layout when Q is
        dense, or (O, LSE) when return_lse.
    """
    head_dim = _check_inputs(Q)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    try:
        code = _CAUSAL_CODES[causal]
    except (KeyError, TypeError):
        raise ValueError(
            f"causal must be False, True, 'top_left' or 'bottom_right', got {causal!r}"
        ) from None
    _check_gqa_heads(Q, K)
    o, lse = _C.flash_attention_forward_ex(Q, K, V, code, float(scale), bool(return_lse),
                                           attn_mask)
    return (o, lse) if return_lse else o


class FlashAttentionFunction(torch.autograd.Function):
    """Differentiable fused attention: the MFMA forward (which also returns the
    row LSE), then the MFMA backward from the saved Q, K, V, O and LSE.

    No reference counterpart: the reference's Function is forward-only
    (reference ops.py:47-52), and so is FlashAttentionSM75Function here.
    """

    @staticmethod
    def forward(ctx, Q, K, V, code, scale, attn_mask):
        O, LSE = _C.flash_attention_forward_ex(Q, K, V, code, scale, True, attn_mask)
        ctx.save_for_backward(Q, K, V, O, LSE)
        ctx.code = code
        ctx.scale = scale
        ctx.attn_mask = attn_mask
        return O

    @staticmethod
    @torch.autograd.function.once_differentiable
    def backward(ctx, dO):
        # The backward kernels are not differentiable themselves: a double
        # backward raises instead of returning wrong second derivatives.
        Q, K, V, O, LSE = ctx.saved_tensors
        dQ, dK, dV = _C.flash_attention_backward(dO, Q, K, V, O, LSE, ctx.code, ctx.scale,
                                                 ctx.attn_mask)
        return dQ, dK, dV, None, None, None


def flash_attention(Q, K, V, causal=False, scale=None, attn_mask=None):
    """Fused attention with a backward pass (training).

    Same inputs as :func:`flash_attention_forward_ex` (fp16 or bf16, grouped
    K/V heads, N_q != N_k, either causal alignment, a boolean ``attn_mask``,
    which is not differentiated).  When
    autograd records the call, the backward computes dQ, dK and dV with the
    fused MFMA kernels (deterministic; for grouped heads dK and dV sum over
    each KV head's query heads).  No reference counterpart.

    Returns:
        O [B, H_q, N_q, D] in Q's dtype.
    """
    head_dim = _check_inputs(Q)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    try:
        code = _CAUSAL_CODES[causal]
    except (KeyError, TypeError):
        raise ValueError(
            f"causal must be False, True, 'top_left' or 'bottom_right', got {causal!r}"
        ) from None
    _check_gqa_heads(Q, K)
    if torch.is_grad_enabled() and (Q.requires_grad or K.requires_grad or V.requires_grad):
        return FlashAttentionFunction.apply(Q, K, V, code, float(scale), attn_mask)
    return _C.flash_attention_forward_ex(Q, K, V, code, float(scale), False, attn_mask)[0]


def flash_attention_backward(dO, Q, K, V, O, LSE, causal=False, scale=None, attn_mask=None):
    """Gradients (dQ, dK, dV) of ``O = flash_attention_forward_ex(Q, K, V,
    causal, scale, attn_mask=attn_mask)`` given dO and that call's LSE
    (``return_lse=True``).

    No reference counterpart.  Deterministic; fp16 or bf16 like the inputs.
    """
    head_dim = _check_inputs(Q)
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    try:
        code = _CAUSAL_CODES[causal]
    except (KeyError, TypeError):
        raise ValueError(
            f"causal must be False, True, 'top_left' or 'bottom_right', got {causal!r}"
        ) from None
    _check_gqa_heads(Q, K)
    return _C.flash_attention_backward(dO, Q, K, V, O, LSE, code, float(scale), attn_mask)
