"""Separate query/key lengths, strided views and the SDPA patch on the GPU.

Parity bar as everywhere: |O - O_ref| <= 2e-3 + 1e-2 |O_ref| against the
numpy oracle (fp32, reference op order) on the same seeded inputs.  For
N_q != N_k the oracle's masks are pinned against torch's CPU SDPA (top-left)
and the tail of the square causal oracle (bottom-right) in test_oracle.py.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from flash_attention_sm75 import flash_attention_forward_ex
from flash_attention_sm75 import sdpa_patch as sp
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def seeded(shape, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g).half()


def assert_parity(out, expect, label):
    out = out.detach().float().cpu().numpy()
    res = ref.check_correctness(out, expect, name=label, atol=ATOL, rtol=RTOL)
    print(f"  {label}: max_abs={res['max_abs_err']:.3e}", flush=True)
    assert res["allclose"], res


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal
    (1, 8, 2, 1, 1000, 128, False),        # decode step
    (3, 4, 4, 1, 77, 64, True),            # decode: top-left sees key 0 only
    (2, 4, 1, 7, 300, 128, "top_left"),
    (2, 4, 1, 7, 300, 128, "bottom_right"),
    (1, 2, 2, 300, 77, 64, "bottom_right"),  # rows 0..222 see no key
    (1, 2, 2, 300, 77, 64, "top_left"),
    (1, 4, 2, 129, 4096, 64, "bottom_right"),  # chunked prefill
    (1, 4, 2, 200, 129, 128, False),
    (2, 8, 8, 64, 64, 128, "bottom_right"),  # equal lengths: same as top-left
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", CASES)
def test_separate_lengths_match_oracle(device, B, Hq, Hkv, Nq, Nk, D, causal):
    print(f"[case] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal}", flush=True)
    q = seeded((B, Hq, Nq, D), 1)
    k = seeded((B, Hkv, Nk, D), 2)
    v = seeded((B, Hkv, Nk, D), 3)
    code = {False: 0, "top_left": 1, True: 1, "bottom_right": 2}[causal]
    o, lse = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                        causal=causal, return_lse=True)
    torch.cuda.synchronize()
    expect = ref.attention_reference(q.numpy(), k.numpy(), v.numpy(), causal=code,
                                     return_f32=True)
    assert_parity(o, expect, f"Nq{Nq} Nk{Nk} c={causal}")
    lse_ref = ref.attention_lse(q.numpy(), k.numpy(), causal=code)
    got = lse.cpu().numpy()
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(got), fin)
    assert np.all(np.isneginf(got[~fin]))
    np.testing.assert_allclose(got[fin], lse_ref[fin], atol=1e-3, rtol=1e-4)


def test_bottom_right_equals_square_tail(device):
    """Property at a larger size: bottom-right Nq < Nk is the tail of the
    square causal launch.  Not bit for bit: the rows fall into different
    waves, whose (wave-uniform) lazy-rescale decisions differ, so the fp32
    sums round differently."""
    Nk, Nq = 2048, 300
    q = seeded((1, 8, Nk, 128), 4).to(device)
    k = seeded((1, 2, Nk, 128), 5).to(device)
    v = seeded((1, 2, Nk, 128), 6).to(device)
    full = flash_attention_forward_ex(q, k, v, causal=True)
    tail = flash_attention_forward_ex(q[:, :, Nk - Nq:], k, v, causal="bottom_right")
    torch.cuda.synchronize()
    diff = (tail.float() - full[:, :, Nk - Nq:].float()).abs()
    assert diff.max().item() <= 2e-3


def test_strided_views_in_place(device):
    """[B, N, H, D] buffers viewed as [B, H, N, D] are read in place and O
    keeps that layout (so transpose(1, 2) of it is contiguous)."""
    B, H, Hkv, N, D = 2, 8, 2, 333, 128
    qb = seeded((B, N, H, D), 7).to(device)
    kb = seeded((B, N, Hkv, D), 8).to(device)
    vb = seeded((B, N, Hkv, D), 9).to(device)
    q, k, v = (t.transpose(1, 2) for t in (qb, kb, vb))
    o = flash_attention_forward_ex(q, k, v, causal=True)
    assert o.transpose(1, 2).is_contiguous()
    o_ref = flash_attention_forward_ex(q.contiguous(), k.contiguous(), v.contiguous(), causal=True)
    torch.cuda.synchronize()
    assert torch.equal(o, o_ref)


def test_unaligned_views_are_copied(device):
    """A view whose row stride is not a multiple of 8 elements is copied
    first and still gives the right answer."""
    base = seeded((1, 2, 40, 72), 10).to(device)
    q = base[..., :64]  # row stride 72: fine (multiple of 8)
    k = seeded((1, 2, 40, 68), 11).to(device)[..., :64]  # row stride 68: copied
    v = seeded((1, 2, 40, 64), 12).to(device)
    o = flash_attention_forward_ex(q, k, v)
    torch.cuda.synchronize()
    expect = ref.attention_reference(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(),
                                     return_f32=True)
    assert_parity(o, expect, "unaligned")


def test_ex_rejects_bad_causal(device):
    q = seeded((1, 1, 4, 64), 13).to(device)
    with pytest.raises(ValueError, match="causal must be"):
        flash_attention_forward_ex(q, q, q, causal="diagonal")


# ---- the SDPA patch ----------------------------------------------------------

@pytest.fixture
def patched():
    sp.apply_patch()
    sp.reset_stats()
    try:
        yield
    finally:
        sp.remove_patch()


def sdpa_ref_cpu(q, k, v, is_causal, scale=None):
    """torch SDPA in fp32 on the CPU (GQA expanded), the parity reference."""
    rep = q.size(1) // k.size(1)
    kf = k.float().cpu().repeat_interleave(rep, dim=1)
    vf = v.float().cpu().repeat_interleave(rep, dim=1)
    return sp._original_sdpa(q.float().cpu(), kf, vf, is_causal=is_causal, scale=scale).numpy()


@pytest.mark.parametrize("Nq,Nk,is_causal", [(128, 128, True), (100, 100, False),
                                             (1, 513, False), (9, 40, True)])
def test_patched_sdpa_matches_fp32_sdpa(device, patched, Nq, Nk, is_causal):
    q = seeded((2, 8, Nq, 64), 20).to(device)
    k = seeded((2, 2, Nk, 64), 21).to(device)
    v = seeded((2, 2, Nk, 64), 22).to(device)
    o = F.scaled_dot_product_attention(q, k, v, is_causal=is_causal, enable_gqa=True)
    torch.cuda.synchronize()
    assert sp._stats["flash"] == 1 and sp._stats["fallback"] == 0
    assert_parity(o, sdpa_ref_cpu(q, k, v, is_causal), f"sdpa Nq{Nq} Nk{Nk}")


@pytest.mark.parametrize("mshape", [(2, 1, 1, 40), (24, 40), (24, 24)])
def test_mask_with_is_causal_behaves_as_unpatched(device, patched, mshape, monkeypatch):
    """A boolean attn_mask together with is_causal=True goes to torch
    unchanged (reason mask_and_causal; reference examples/
    llama_attention_replacement.py:61-77 passes every masked call through):
    the patched call hands torch's own function exactly its arguments (the same
    tensor objects, the same keywords), once, and raises what the unpatched
    call raises.  Torch documents the pair as an error; where its GPU path
    returns instead, the values are not a reference (over a seeded sweep some
    of them hold mask-like 0 / -inf entries, and consecutive calls can
    differ), so they are not compared."""
    nk = mshape[-1]
    print(f"[case] mask {mshape} with is_causal", flush=True)
    q = seeded((2, 4, 24, 64), 30).to(device)
    k = seeded((2, 4, nk, 64), 31).to(device)
    g = torch.Generator("cpu").manual_seed(32)
    m = (torch.rand(*mshape, generator=g) < 0.7).to(device)
    real = sp._original_sdpa
    calls = []

    def spy(*args, **kwargs):
        calls.append((args, kwargs))
        return real(*args, **kwargs)

    monkeypatch.setattr(sp, "_original_sdpa", spy)
    outcome = []
    for fn in (F.scaled_dot_product_attention, real, real):
        try:
            outcome.append(fn(q, k, k, attn_mask=m, is_causal=True))
        except RuntimeError as e:
            outcome.append((type(e).__name__, str(e)))
    torch.cuda.synchronize()
    s = sp.patch_stats()
    assert (s["flash"], s["fallback"], s["fallback_reasons"]) == (0, 1, {"mask_and_causal": 1})
    assert len(calls) == 1, calls
    (args, kwargs), = calls
    assert len(args) == 3 and args[0] is q and args[1] is k and args[2] is k
    assert kwargs.pop("attn_mask") is m
    assert kwargs == dict(dropout_p=0.0, is_causal=True, scale=None), kwargs
    kinds = [isinstance(o, tuple) for o in outcome]
    assert kinds[0] == kinds[1] == kinds[2], outcome
    if kinds[0]:
        print(f"  torch raises: {outcome[0][0]}", flush=True)
        assert outcome[0] == outcome[1] == outcome[2]
    else:
        print("  torch returns (the pair's values are undefined): pass-through checked", flush=True)


def test_patched_sdpa_fallbacks(device, patched):
    q = seeded((1, 4, 16, 64), 23).to(device)
    cases = {
        "not_fp16": (q.float(), q.float(), q.float(), {}),
        "head_dim_unsupported": (q[..., :32].contiguous(),) * 3 + ({},),
        "has_attn_mask": (q, q, q, dict(attn_mask=torch.zeros(16, 16, device=device,
                                                               dtype=torch.float16))),
    }
    for reason, (a, b, c, kw) in cases.items():
        got = F.scaled_dot_product_attention(a, b, c, **kw)
        want = sp._original_sdpa(a, b, c, **kw)
        assert torch.equal(got, want), reason
    reasons = sp._stats["fallback_reasons"]
    for r in ("not_fp16", "head_dim_unsupported", "has_attn_mask"):
        assert reasons.get(r) == 1, (r, reasons)
    assert sp._stats["flash"] == 0


def tiny_qwen2(head_dim, layers=2, seed=0):
    transformers = pytest.importorskip("transformers")
    heads, kv = (4, 2) if head_dim == 64 else (4, 1)
    cfg = transformers.Qwen2Config(
        vocab_size=2000, hidden_size=heads * head_dim, intermediate_size=512,
        num_hidden_layers=layers, num_attention_heads=heads, num_key_value_heads=kv,
        max_position_embeddings=4096, attn_implementation="sdpa")
    torch.manual_seed(seed)
    return transformers, transformers.Qwen2ForCausalLM(cfg).half().to("cuda").eval()


def compare_logits(plain, patched_logits, label):
    """Last-token logits: close in value, and the same top-1 whenever the
    unpatched top-1 wins by more than twice the observed difference (a
    random-init model can have near ties, which no kernel must be held to)."""
    a = plain.float()
    b = patched_logits.float()
    diff = (a - b).abs().max().item()
    scale = a.abs().max().item()
    print(f"  {label}: max |dlogit| = {diff:.3e} (max |logit| {scale:.3e})", flush=True)
    assert diff <= 1e-3 + 2e-2 * scale
    top2 = a.topk(2, dim=-1)
    margin = top2.values[..., 0] - top2.values[..., 1]
    decided = margin > 2 * diff
    assert torch.equal(a.argmax(-1)[decided], b.argmax(-1)[decided])


@pytest.mark.parametrize("head_dim", [64, 128])
def test_tiny_qwen2_prefill_and_decode(device, head_dim):
    """The reference's prefill check (tests/test_prefill_correctness.py:37-72)
    on a random-init Qwen2 of the same architecture, plus teacher-forced
    KV-cache decode steps, which now also run on the kernel (N_q = 1)."""
    transformers, model = tiny_qwen2(head_dim)
    g = torch.Generator("cpu").manual_seed(head_dim)
    ids = torch.randint(0, 2000, (2, 300), generator=g).to(device)
    prompt, steps = ids[:, :280], ids[:, 280:]

    def run():
        with torch.no_grad():
            out = model(input_ids=prompt, use_cache=True)
            logits = [out.logits[:, -1]]
            cache = out.past_key_values
            for t in range(steps.size(1)):
                out = model(input_ids=steps[:, t:t + 1], past_key_values=cache, use_cache=True)
                cache = out.past_key_values
                logits.append(out.logits[:, -1])
        return torch.stack(logits, 1)

    plain = run()
    sp.apply_patch()
    sp.reset_stats()
    try:
        pat = run()
        stats = sp.patch_stats()
    finally:
        sp.remove_patch()
    torch.cuda.synchronize()
    print(f"  stats: {stats}", flush=True)
    assert stats["fallback"] == 0
    assert stats["flash"] == 2 * (1 + steps.size(1))
    compare_logits(plain[:, 0], pat[:, 0], f"prefill d{head_dim}")
    compare_logits(plain[:, 1:], pat[:, 1:], f"decode d{head_dim}")


def test_patched_training_step(device):
    """One training step of a random-init Qwen2 (fp16) through the patch: every
    attention call runs on the kernels, forward and backward (the patch routes
    calls that need gradients to flash_attention), and the loss and every
    parameter gradient agree with torch's own SDPA in the same dtype
    (relative L2 difference below 3e-2; both runs round the rest of the model
    identically, so the difference is the attention's rounding)."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(
        vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
        attn_implementation="sdpa")
    torch.manual_seed(0)
    model = transformers.Qwen2ForCausalLM(cfg).half().to("cuda").train()
    ids = torch.randint(0, 1000, (2, 200), generator=torch.Generator("cpu").manual_seed(3))
    ids = ids.to(device)

    def step():
        model.zero_grad(set_to_none=True)
        out = model(input_ids=ids, labels=ids)
        out.loss.backward()
        torch.cuda.synchronize()
        return out.loss.detach().float().item(), {
            n: p.grad.detach().float().clone()
            for n, p in model.named_parameters() if p.grad is not None}

    loss0, g0 = step()
    sp.apply_patch()
    sp.reset_stats()
    try:
        loss1, g1 = step()
        stats = sp.patch_stats()
    finally:
        sp.remove_patch()
    print(f"  stats {stats}; loss {loss0:.5f} vs {loss1:.5f}", flush=True)
    assert stats["fallback"] == 0 and stats["flash"] == cfg.num_hidden_layers
    assert abs(loss0 - loss1) <= 1e-3 * abs(loss0)
    worst = max(((g1[n] - g0[n]).norm() / g0[n].norm()).item() for n in g0)
    print(f"  worst relative gradient difference {worst:.2e}", flush=True)
    assert g0.keys() == g1.keys() and worst < 3e-2


def test_patched_training_step_padded_batch(device):
    """A training step on a right-padded batch: transformers hands SDPA a
    boolean padding-and-causal mask, so the forward and the masked backward
    both run on the kernels; loss and parameter gradients agree with torch's
    SDPA in the same dtype (relative L2 below 3e-2)."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(
        vocab_size=1000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=1024,
        attn_implementation="sdpa")
    torch.manual_seed(1)
    model = transformers.Qwen2ForCausalLM(cfg).half().to("cuda").train()
    g = torch.Generator("cpu").manual_seed(4)
    ids = torch.randint(0, 1000, (2, 192), generator=g)
    attn = torch.ones(2, 192, dtype=torch.long)
    attn[1, 130:] = 0  # second sequence right-padded after 130 tokens
    labels = ids.clone()
    labels[attn == 0] = -100
    ids, attn, labels = ids.to(device), attn.to(device), labels.to(device)

    def step():
        model.zero_grad(set_to_none=True)
        out = model(input_ids=ids, attention_mask=attn, labels=labels)
        out.loss.backward()
        torch.cuda.synchronize()
        return out.loss.detach().float().item(), {
            n: p.grad.detach().float().clone()
            for n, p in model.named_parameters() if p.grad is not None}

    loss0, g0 = step()
    sp.apply_patch()
    sp.reset_stats()
    try:
        loss1, g1 = step()
        stats = sp.patch_stats()
    finally:
        sp.remove_patch()
    print(f"  stats {stats}; loss {loss0:.5f} vs {loss1:.5f}", flush=True)
    assert stats["fallback"] == 0 and stats["flash"] == cfg.num_hidden_layers
    assert abs(loss0 - loss1) <= 1e-3 * abs(loss0)
    worst = max(((g1[n] - g0[n]).norm() / g0[n].norm()).item() for n in g0)
    print(f"  worst relative gradient difference {worst:.2e}", flush=True)
    assert g0.keys() == g1.keys() and worst < 3e-2
