"""SDPA monkey-patch host logic (no GPU): install/remove, pass-through of
every call the kernel cannot take, and statistics, mirroring reference
examples/llama_attention_replacement.py:18-119."""
import pytest
import torch
import torch.nn.functional as F

from flash_attention_sm75 import sdpa_patch as sp


@pytest.fixture
def patched():
    sp.apply_patch()
    sp.reset_stats()
    try:
        yield
    finally:
        sp.remove_patch()


def test_apply_and_remove_swap_the_function():
    orig = F.scaled_dot_product_attention
    assert orig is sp._original_sdpa
    sp.apply_patch()
    try:
        assert F.scaled_dot_product_attention is sp._patched_sdpa
        assert torch.nn.functional.scaled_dot_product_attention is sp._patched_sdpa
        sp.apply_patch()  # idempotent
        assert sp.patch_stats()["active"] is True
    finally:
        sp.remove_patch()
    assert F.scaled_dot_product_attention is orig
    assert sp.patch_stats()["active"] is False


def test_reference_module_name_reexports():
    import llama_attention_replacement as lar
    assert lar.apply_patch is sp.apply_patch and lar._stats is sp._stats


@pytest.mark.parametrize("kw", [dict(), dict(is_causal=True), dict(scale=0.3),
                                dict(attn_mask=torch.zeros(5, 7))])
def test_cpu_calls_pass_through_unchanged(patched, kw):
    g = torch.Generator().manual_seed(0)
    q = torch.randn(2, 4, 5, 64, generator=g)
    k = torch.randn(2, 4, 7, 64, generator=g)
    v = torch.randn(2, 4, 7, 64, generator=g)
    got = F.scaled_dot_product_attention(q, k, v, **kw)
    want = sp._original_sdpa(q, k, v, **kw)
    assert torch.equal(got, want)
    s = sp.patch_stats()
    assert (s["total"], s["flash"], s["fallback"]) == (1, 0, 1)
    assert s["fallback_reasons"] == {"not_cuda": 1}


def test_fallback_keeps_extra_kwargs(patched):
    q = torch.randn(1, 4, 3, 64)
    k = torch.randn(1, 2, 3, 64)
    v = torch.randn(1, 2, 3, 64)
    got = F.scaled_dot_product_attention(q, k, v, enable_gqa=True)
    assert torch.equal(got, sp._original_sdpa(q, k, v, enable_gqa=True))


def test_tiny_qwen2_on_cpu_is_unchanged(patched):
    """A random-init Qwen2 (no weights are downloadable here): every attention
    call of the CPU model falls back, so the logits are bit-identical."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(
        vocab_size=500, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
        num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=512,
        attn_implementation="sdpa")
    torch.manual_seed(0)
    model = transformers.Qwen2ForCausalLM(cfg).eval()
    ids = torch.randint(0, 500, (1, 20))
    with torch.no_grad():
        patched_logits = model(input_ids=ids).logits
        sp.remove_patch()
        plain = model(input_ids=ids).logits
        sp.apply_patch()
    assert torch.equal(patched_logits, plain)
    assert sp._stats["fallback_reasons"].get("not_cuda") == 2


class _DeviceTensor:
    """Stand-in for a device tensor in the eligibility check (no GPU here):
    the shape, dtype and device facts _fallback_reason reads."""

    def __init__(self, *shape, dtype=torch.float16):
        self.shape, self.dtype, self.is_cuda = torch.Size(shape), dtype, True

    def dim(self):
        return len(self.shape)

    def size(self, i):
        return self.shape[i]


@pytest.mark.parametrize("kwargs,reason", [({}, "gqa_not_enabled"),
                                           ({"enable_gqa": False}, "gqa_not_enabled"),
                                           ({"enable_gqa": True}, None)])
def test_grouped_heads_need_enable_gqa(kwargs, reason):
    """torch's SDPA rejects Hq != Hkv unless enable_gqa=True, so the patch
    must not silently compute grouped-query attention for such a call."""
    q, k = _DeviceTensor(1, 8, 16, 64), _DeviceTensor(1, 2, 16, 64)
    assert sp._fallback_reason(q, k, k, None, 0.0, False, kwargs) == reason
    same = _DeviceTensor(1, 8, 16, 64)
    assert sp._fallback_reason(q, same, same, None, 0.0, False, {}) is None


def test_gqa_without_enable_gqa_raises_like_torch(patched):
    q, k = torch.randn(1, 4, 3, 64), torch.randn(1, 2, 3, 64)
    with pytest.raises(RuntimeError):
        sp._original_sdpa(q, k, k)
    with pytest.raises(RuntimeError):
        F.scaled_dot_product_attention(q, k, k)


class _DeviceMask(_DeviceTensor):
    def __init__(self, *shape):
        super().__init__(*shape, dtype=torch.bool)


def test_mask_with_is_causal_goes_to_torch():
    """A boolean mask together with is_causal=True is left to torch, which
    documents the pair as an error (reference examples/
    llama_attention_replacement.py:61-77 passes every masked call through):
    the patched call then raises or returns exactly what the unpatched one
    does.  Either flag alone stays on the kernel."""
    q = _DeviceTensor(1, 4, 16, 64)
    m = _DeviceMask(1, 1, 16, 16)
    assert sp._fallback_reason(q, q, q, m, 0.0, True, {}) == "mask_and_causal"
    assert sp._fallback_reason(q, q, q, m, 0.0, False, {}) is None
    assert sp._fallback_reason(q, q, q, None, 0.0, True, {}) is None


def test_mask_with_is_causal_on_cpu_matches_unpatched(patched):
    q = torch.randn(1, 2, 6, 64)
    m = torch.rand(6, 6) < 0.7
    outcome = []
    for fn in (F.scaled_dot_product_attention, sp._original_sdpa):
        try:
            outcome.append(fn(q, q, q, attn_mask=m, is_causal=True))
        except RuntimeError as e:
            outcome.append((type(e), str(e)))
    if isinstance(outcome[1], tuple):
        assert outcome[0] == outcome[1]
    else:
        assert torch.equal(outcome[0], outcome[1])
