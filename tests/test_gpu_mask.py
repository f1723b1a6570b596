"""Explicit boolean attn_mask on the GPU (prefill and split-K paths).

No reference counterpart (the reference rejects masked SDPA calls); the
oracle's masking is pinned against torch's CPU SDPA in test_oracle.py.  Bar
as everywhere: |O - O_ref| <= 2e-3 + 1e-2 |O_ref| on the same seeded inputs;
LSE against the float64 closed form.  Rows that see no key: O = 0 and
LSE = -inf (torch SDPA gives NaN there).
"""
import ctypes

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from capi_types import LIB
from flash_attention_sm75 import flash_attention_forward_ex
from flash_attention_sm75 import sdpa_patch as sp
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def seeded(shape, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g).half()


def rand_mask(shape, p, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.rand(*shape, generator=g) < p


def assert_parity(out, expect, label):
    res = ref.check_correctness(out.float().cpu().numpy(), expect, name=label, atol=ATOL, rtol=RTOL)
    print(f"  {label}: max_abs={res['max_abs_err']:.3e}", flush=True)
    assert res["allclose"], res


def test_pack_mask_bits(device):
    """fa_sm75_pack_mask against numpy: bit k of word w = element 64 w + k."""
    lib = ctypes.CDLL(LIB)
    f = lib.fa_sm75_pack_mask
    f.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int
    m = rand_mask((2, 3, 5, 200), 0.5, 1)
    md = m.to(device)
    words = (200 + 63) // 64
    out = torch.full((2, 3, 5, words), -1, dtype=torch.int64, device=device)
    st = md.stride()
    assert f(md.data_ptr(), 2, 3, 5, 200, st[0], st[1], st[2], st[3], out.data_ptr(),
             torch.cuda.current_stream().cuda_stream) == 0
    # a transposed (strided) view of the same mask
    mt = m.transpose(2, 3).contiguous().transpose(2, 3).to(device)
    out2 = torch.full_like(out, -1)
    st = mt.stride()
    assert f(mt.data_ptr(), 2, 3, 5, 200, st[0], st[1], st[2], st[3], out2.data_ptr(),
             torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    padded = np.zeros((2, 3, 5, words * 64), dtype=np.uint8)
    padded[..., :200] = m.numpy()
    want = np.packbits(padded.reshape(2, 3, 5, words, 64), axis=-1, bitorder="little")
    want = want.view(np.uint64).reshape(2, 3, 5, words)
    assert np.array_equal(out.cpu().numpy().view(np.uint64), want)
    assert np.array_equal(out2.cpu().numpy().view(np.uint64), want)


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, mask shape (broadcast), p(visible), causal
    (2, 4, 2, 300, 300, 128, (2, 4, 300, 300), 0.6, False),
    (2, 4, 2, 300, 300, 64, (2, 1, 300, 300), 0.9, True),
    (1, 8, 8, 257, 511, 128, (257, 511), 0.3, False),
    (3, 4, 1, 200, 200, 64, (3, 1, 1, 200), 0.8, False),  # key padding
    (2, 8, 2, 1, 5000, 128, (2, 1, 1, 5000), 0.7, False),  # decode + padding
    (2, 8, 2, 4, 3000, 64, (2, 8, 4, 3000), 0.5, "bottom_right"),  # split-K, per-head mask
    (1, 4, 4, 100, 100, 128, (100, 100), 0.02, False),  # sparse: empty rows
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,mshape,p,causal", CASES)
def test_masked_forward_matches_oracle(device, B, Hq, Hkv, Nq, Nk, D, mshape, p, causal):
    print(f"[case] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} mask={mshape} p={p} "
          f"causal={causal}", flush=True)
    q = seeded((B, Hq, Nq, D), 2)
    k = seeded((B, Hkv, Nk, D), 3)
    v = seeded((B, Hkv, Nk, D), 4)
    m = rand_mask(mshape, p, 5)
    o, lse = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device), causal=causal,
                                        return_lse=True, attn_mask=m.to(device))
    torch.cuda.synchronize()
    code = {False: 0, True: 1, "bottom_right": 2}[causal]
    expect = ref.attention_reference_chunked(q.numpy(), k.numpy(), v.numpy(), causal=code,
                                             attn_mask=m.numpy(), return_f32=True)
    assert_parity(o, expect, "masked")
    want = ref.attention_lse(q.numpy(), k.numpy(), causal=code, attn_mask=m.numpy())
    got = lse.cpu().numpy()
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    np.testing.assert_allclose(got[fin], want[fin], atol=1e-3, rtol=1e-4)


def test_all_true_mask_equals_no_mask(device):
    q, k, v = (seeded((2, 8, 333, 128), s).to(device) for s in (6, 7, 8))
    ones = torch.ones(333, 333, dtype=torch.bool, device=device)
    a = flash_attention_forward_ex(q, k, v, attn_mask=ones)
    b = flash_attention_forward_ex(q, k, v)
    tril = torch.ones(333, 333, dtype=torch.bool, device=device).tril()
    c = flash_attention_forward_ex(q, k, v, attn_mask=tril)
    d = flash_attention_forward_ex(q, k, v, causal=True)
    torch.cuda.synchronize()
    assert torch.equal(a, b)   # same kernel path bits, mask never hides anything
    assert (c.float() - d.float()).abs().max().item() <= 2e-3


def test_patched_sdpa_bool_mask(device):
    sp.apply_patch()
    sp.reset_stats()
    try:
        q = seeded((2, 8, 64, 64), 9).to(device)
        k = seeded((2, 2, 96, 64), 10).to(device)
        v = seeded((2, 2, 96, 64), 11).to(device)
        m = rand_mask((2, 1, 64, 96), 0.7, 12)
        m[..., 0] = True
        o = F.scaled_dot_product_attention(q, k, v, attn_mask=m.to(device), enable_gqa=True)
        fm = torch.zeros(64, 96, dtype=torch.float16, device=device)
        F.scaled_dot_product_attention(q, k, v, attn_mask=fm, enable_gqa=True)
        torch.cuda.synchronize()
        assert sp._stats["flash"] == 1
        assert sp._stats["fallback_reasons"] == {"has_attn_mask": 1}
    finally:
        sp.remove_patch()
    rep = 4
    want = sp._original_sdpa(q.float().cpu(), k.float().cpu().repeat_interleave(rep, 1),
                             v.float().cpu().repeat_interleave(rep, 1), attn_mask=m).numpy()
    assert_parity(o, want, "sdpa bool mask")


def test_tiny_qwen2_left_padded_batch(device):
    """A padded batch (left padding, transformers' boolean SDPA masks):
    prefill and teacher-forced decode logits of the real tokens, patched vs
    unpatched, on a random-init Qwen2."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(
        vocab_size=2000, hidden_size=256, intermediate_size=512, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096,
        attn_implementation="sdpa")
    torch.manual_seed(0)
    model = transformers.Qwen2ForCausalLM(cfg).half().to(device).eval()
    g = torch.Generator("cpu").manual_seed(13)
    ids = torch.randint(0, 2000, (3, 150), generator=g)
    lens = [150, 97, 40]
    attn = torch.zeros(3, 150, dtype=torch.long)
    for i, n in enumerate(lens):
        attn[i, 150 - n:] = 1
    ids, attn = ids.to(device), attn.to(device)
    steps = torch.randint(0, 2000, (3, 6), generator=g).to(device)

    def run():
        with torch.no_grad():
            out = model(input_ids=ids, attention_mask=attn, use_cache=True)
            logits = [out.logits[:, -1]]
            cache, am = out.past_key_values, attn
            for t in range(steps.size(1)):
                am = torch.cat([am, torch.ones(3, 1, dtype=am.dtype, device=device)], 1)
                out = model(input_ids=steps[:, t:t + 1], attention_mask=am, past_key_values=cache,
                            use_cache=True)
                cache = out.past_key_values
                logits.append(out.logits[:, -1])
        return torch.stack(logits, 1).float()

    plain = run()
    sp.apply_patch()
    sp.reset_stats()
    try:
        pat = run()
        stats = sp.patch_stats()
    finally:
        sp.remove_patch()
    print(f"  stats: {stats}", flush=True)
    assert stats["flash"] > 0
    diff = (plain - pat).abs().max().item()
    scale = plain.abs().max().item()
    print(f"  max |dlogit| = {diff:.3e} (max |logit| {scale:.3e})", flush=True)
    assert diff <= 1e-3 + 2e-2 * scale
