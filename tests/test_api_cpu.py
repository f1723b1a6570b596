"""Host-side behaviour of the Python API and the binding, without a GPU.

Every validation in the reference API runs before any device work
(reference src/flash_attention_sm75/ops.py:55-82,
src/bindings/pytorch_extension.cpp:21-26,52-68), and so do ours; these tests
force each error from the host.
"""
import pytest
import torch

import flash_attn_sm75_cuda as _C
import flash_attention_sm75 as fa
from flash_attention_sm75 import flash_attention_forward
from flash_attention_sm75 import ops


def h(*shape):
    return torch.zeros(*shape, dtype=torch.float16)


def test_public_surface():
    assert fa.__version__ == "0.1.0"
    assert "flash_attention_forward" in fa.__all__
    for name in ("naive_attention_forward", "flash_attention_forward",
                 "flash_attention_forward_scalar", "flash_attention_forward_wmma_qk",
                 "flash_attention_forward_lse"):
        assert hasattr(_C, name), name


def test_rank_check():
    with pytest.raises(ValueError, match=r"Q must be 4D \[B, H, N, D\]"):
        flash_attention_forward(h(8, 128, 64), h(8, 128, 64), h(8, 128, 64))


def test_head_dim_check():
    # reference tests/test_api.py:20-29
    q = h(1, 8, 128, 96)
    with pytest.raises(RuntimeError, match="supports head_dim=64 or 128"):
        flash_attention_forward(q, q, q)


def test_gqa_divisibility_message():
    with pytest.raises(RuntimeError, match=r"GQA expansion: Q heads \(6\) not divisible by K/V heads \(4\)"):
        flash_attention_forward(h(1, 6, 16, 64), h(1, 4, 16, 64), h(1, 4, 16, 64))


def test_expand_kv_helper():
    q, k, v = h(1, 8, 4, 64), torch.randn(1, 2, 4, 64).half(), torch.randn(1, 2, 4, 64).half()
    k2, v2 = ops._expand_kv_for_gqa(q, k, v)
    assert k2.shape == (1, 8, 4, 64)
    assert torch.equal(k2[:, 5], k[:, 1]) and torch.equal(v2[:, 3], v[:, 0])
    k3, _ = ops._expand_kv_for_gqa(q, h(1, 8, 4, 64), h(1, 8, 4, 64))
    assert k3.shape == (1, 8, 4, 64)


def test_backward_message():
    # reference tests/test_api.py:31-41 expects this substring
    with pytest.raises(NotImplementedError, match="Backward pass is not implemented"):
        ops.FlashAttentionSM75Function.backward(None, h(1, 1, 1, 64))


@pytest.mark.parametrize("op", ["flash_attention_forward", "naive_attention_forward",
                                "flash_attention_forward_scalar",
                                "flash_attention_forward_wmma_qk",
                                "flash_attention_forward_lse"])
def test_binding_rejects_host_tensors(op):
    q = h(1, 1, 16, 64)
    with pytest.raises(RuntimeError, match="Q must be a CUDA tensor"):
        getattr(_C, op)(q, q, q, False, 0.125)


def test_binding_signature_is_reference_shaped():
    q = h(1, 1, 16, 64)
    with pytest.raises(TypeError):
        _C.flash_attention_forward(q, q, q)  # causal and scale are required


def test_product_path_has_no_oracle_import():
    import sys

    import flash_attention_sm75.ops as m

    src = open(m.__file__).read()
    assert "oracle" not in src
    assert not any(name == "oracle" or name.startswith("oracle.") for name in
                   getattr(m, "__dict__", {}))
    del sys


def test_training_surface():
    """The added differentiable entry points (no reference counterpart)."""
    for name in ("flash_attention", "flash_attention_backward"):
        assert name in fa.__all__ and callable(getattr(fa, name))
    assert hasattr(_C, "flash_attention_backward")


def test_flash_attention_argument_checks():
    from flash_attention_sm75 import flash_attention, flash_attention_backward

    with pytest.raises(ValueError, match=r"Q must be 4D"):
        flash_attention(h(8, 128, 64), h(8, 128, 64), h(8, 128, 64))
    with pytest.raises(RuntimeError, match="supports head_dim=64 or 128"):
        flash_attention(h(1, 2, 8, 96), h(1, 2, 8, 96), h(1, 2, 8, 96))
    with pytest.raises(ValueError, match="causal must be"):
        flash_attention(h(1, 2, 8, 64), h(1, 2, 8, 64), h(1, 2, 8, 64), causal="diagonal")
    with pytest.raises(RuntimeError, match=r"GQA expansion: Q heads \(6\)"):
        flash_attention(h(1, 6, 8, 64), h(1, 4, 8, 64), h(1, 4, 8, 64))
    q = h(1, 2, 8, 64)
    lse = torch.zeros(1, 2, 8)
    with pytest.raises(RuntimeError, match="inputs must be CUDA tensors"):
        flash_attention_backward(q, q, q, q, q, lse)


def test_backward_binding_checks_before_device():
    q = h(1, 2, 8, 64)
    with pytest.raises(RuntimeError, match="inputs must be CUDA tensors"):
        _C.flash_attention_backward(q, q, q, q, q, torch.zeros(1, 2, 8), 0, 0.125)
    with pytest.raises(TypeError):
        _C.flash_attention_backward(q, q, q, q, q, torch.zeros(1, 2, 8))  # causal, scale required
