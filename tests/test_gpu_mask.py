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


@pytest.mark.parametrize("nk,off", [(1, 0), (17, 5), (1000, 3), (1024, 0), (1025, 7), (2049, 3),
                                    (4097, 0), (5000, 5)])
def test_pack_mask_rows_unaligned(device, nk, off):
    """Rows of consecutive bytes at any alignment and length (16-byte loads,
    one or two 1024-byte chunks per pass, the row's last partial 16 bytes one
    by one) against numpy."""
    lib = ctypes.CDLL(LIB)
    f = lib.fa_sm75_pack_mask
    f.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int
    B, Nq = 2, 3
    g = torch.Generator("cpu").manual_seed(nk + off)
    base = torch.rand(B * Nq * nk + off + 16, generator=g) < 0.5
    m = base[off:off + B * Nq * nk].view(B, 1, Nq, nk)
    md = base.to(device)[off:off + B * Nq * nk].view(B, 1, Nq, nk)
    words = (nk + 63) // 64
    out = torch.full((B, 1, Nq, words), -1, dtype=torch.int64, device=device)
    st = md.stride()
    assert f(md.data_ptr(), B, 1, Nq, nk, st[0], 0, st[2], st[3], out.data_ptr(),
             torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    padded = np.zeros((B, 1, Nq, words * 64), dtype=np.uint8)
    padded[..., :nk] = m.numpy()
    want = np.packbits(padded.reshape(B, 1, Nq, words, 64), axis=-1, bitorder="little")
    assert np.array_equal(out.cpu().numpy().view(np.uint64), want.view(np.uint64).reshape(out.shape))


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, mask shape (broadcast), p(visible), causal
    (2, 4, 2, 300, 300, 128, (2, 4, 300, 300), 0.6, False),
    (2, 4, 2, 300, 300, 64, (2, 1, 300, 300), 0.9, True),
    (1, 8, 8, 257, 511, 128, (257, 511), 0.3, False),
    (3, 4, 1, 200, 200, 64, (3, 1, 1, 200), 0.8, False),  # key padding
    (2, 8, 2, 1, 5000, 128, (2, 1, 1, 5000), 0.7, False),  # decode + padding
    (2, 8, 2, 4, 3000, 64, (2, 8, 4, 3000), 0.5, "bottom_right"),  # split-K, per-head mask
    (1, 4, 4, 100, 100, 128, (100, 100), 0.02, False),  # sparse: empty rows
    (2, 8, 2, 1, 3000, 64, (3000,), 0.6, False),  # 1-D key mask (key bytes, decode)
    (2, 4, 4, 130, 700, 128, (1, 700), 0.7, True),  # [1, Nk] (key bytes, prefill)
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


@pytest.mark.parametrize("D,causal,mshape", [
    (128, True, (2, 1, 700, 700)),
    (64, "bottom_right", (2, 4, 500, 900)),
    (64, True, (2, 1, 700, 700)),
    (128, False, (700, 700)),
])
def test_masked_wide_matches_narrow(device, D, causal, mshape):
    """Mask bits (packed with ranges by the binding) with and without the
    causal flag on 256-row workgroups (policy WIDE): bitwise equal to the
    128-row kernel (policy NARROW) and within the oracle's bar."""
    import flash_attn_sm75_cuda as _C
    B, Hq, Hkv = 2, 4, 2
    Nq, Nk = mshape[-2], mshape[-1]
    print(f"[wide mask] D={D} causal={causal} mask={mshape}", flush=True)
    q, k, v = seeded((B, Hq, Nq, D), 21), seeded((B, Hkv, Nk, D), 22), seeded((B, Hkv, Nk, D), 23)
    m = rand_mask(mshape, 0.8, 24)
    outs = {}
    try:
        for pol in (2, 1):
            _C.set_kernel_policy(pol)
            outs[pol] = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                                   causal=causal, return_lse=True,
                                                   attn_mask=m.to(device))
    finally:
        _C.set_kernel_policy(0)
    torch.cuda.synchronize()
    assert torch.equal(outs[2][0], outs[1][0]) and torch.equal(outs[2][1], outs[1][1])
    code = {False: 0, True: 1, "bottom_right": 2}[causal]
    expect = ref.attention_reference_chunked(q.numpy(), k.numpy(), v.numpy(), causal=code,
                                             attn_mask=m.numpy(), return_f32=True)
    assert_parity(outs[2][0], expect, "wide masked")


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


def test_strided_key_padding_view(device):
    """A [B, 1, 1, Nk] key-padding view with key stride 2 (every other
    column of a wider buffer) is read in place as key bytes."""
    B, Hq, Hkv, Nq, Nk, D = 2, 8, 2, 1, 2500, 128
    q, k, v = seeded((B, Hq, Nq, D), 41), seeded((B, Hkv, Nk, D), 42), seeded((B, Hkv, Nk, D), 43)
    wide = rand_mask((B, 1, 1, 2 * Nk), 0.7, 44)
    m = wide[..., ::2]
    for nq in (1, 200):  # split-K and prefill kernels
        qq = seeded((B, Hq, nq, D), 45)
        o = flash_attention_forward_ex(qq.to(device), k.to(device), v.to(device),
                                       attn_mask=wide.to(device)[..., ::2])
        torch.cuda.synchronize()
        expect = ref.attention_reference(qq.numpy(), k.numpy(), v.numpy(),
                                         attn_mask=m.numpy(), return_f32=True)
        assert_parity(o, expect, f"strided key mask nq={nq}")


KEY_BYTE_CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal, bf16, batch-broadcast, key stride
    (4, 32, 8, 1, 8192, 128, 0, False, False, 1),   # decode, splits + combine
    (2, 14, 2, 1, 3001, 64, 0, True, False, 1),     # Qwen2-0.5B heads, bf16
    (3, 8, 8, 2, 77, 64, 1, False, True, 1),        # top-left decode, broadcast batch
    (1, 4, 4, 512, 512, 128, 0, False, False, 3),   # small launch, strided key bytes
    (2, 8, 2, 300, 700, 128, 2, False, False, 1),   # prefill kernel, bottom-right
    (1, 8, 2, 1000, 1000, 64, 1, True, False, 2),   # prefill, bf16, causal
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal,bf16,bcast,sk", KEY_BYTE_CASES)
def test_key_bytes_equal_packed_bits(device, B, Hq, Hkv, Nq, Nk, D, causal, bf16, bcast, sk):
    """Through the C ABI: a key-padding mask given as bytes (mask_keys, read
    in place) and the same mask packed into bit rows (mask_bits) give the
    same O and LSE bit for bit, with and without a split-K workspace."""
    from capi_types import Params
    print(f"[key bytes] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal} "
          f"bf16={bf16} bcast={bcast} sk={sk}", flush=True)
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_forward.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.restype = ctypes.c_int64
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    pack = lib.fa_sm75_pack_mask
    pack.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p, ctypes.c_void_p]
    dt = torch.bfloat16 if bf16 else torch.float16
    g = torch.Generator("cpu").manual_seed(B * 1000 + Nk)
    q = torch.randn(B, Hq, Nq, D, generator=g).to(dt).to(device)
    k = torch.randn(B, Hkv, Nk, D, generator=g).to(dt).to(device)
    v = torch.randn(B, Hkv, Nk, D, generator=g).to(dt).to(device)
    mb = 1 if bcast else B
    keys = (torch.rand(mb, Nk * sk, generator=g) < 0.7).to(device)  # [mb, Nk*sk] bytes
    keys[:, 0] = True
    kview = keys[:, ::sk]
    words = (Nk + 63) // 64
    bits = torch.empty(mb, 1, 1, words, dtype=torch.int64, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    assert pack(kview.data_ptr(), mb, 1, 1, Nk, kview.stride(0), 0, 0, kview.stride(1),
                bits.data_ptr(), stream) == 0

    def run(use_bytes, with_ws):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((B, Hq, Nq), float("nan"), device=device)
        p = Params()
        p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
        p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = B, Hq, Hkv, Nq, D
        p.seq_len_kv = Nk
        lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
        p.scale, p.causal, p.dtype = D ** -0.5, causal, 1 if bf16 else 0
        p.stream = stream
        if use_bytes:
            p.mask_keys = kview.data_ptr()
            p.mask_keys_stride_b = kview.stride(0) if mb > 1 else 0
            p.mask_keys_stride_k = kview.stride(1)
        else:
            p.mask_bits = bits.data_ptr()
            p.mask_stride_b = words if mb > 1 else 0
        ws = None
        if with_ws:
            n = lib.fa_sm75_workspace_size(ctypes.byref(p))
            if n > 0:
                ws = torch.empty(n, dtype=torch.uint8, device=device)
                p.workspace, p.workspace_bytes = ws.data_ptr(), n
        assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
        torch.cuda.synchronize()
        return o, lse

    for with_ws in (True, False):
        ob, lb = run(True, with_ws)
        op, lp = run(False, with_ws)
        assert torch.equal(ob, op), f"O differs (workspace={with_ws})"
        assert torch.equal(lb, lp), f"LSE differs (workspace={with_ws})"
    npf = lambda t: t.float().cpu().numpy()
    m_np = kview.cpu().numpy()[:, None, None, :]
    if bf16:
        want = ref.attention_f64(npf(q), npf(k), npf(v), causal=causal, attn_mask=m_np)
        spv = ref.attention_f64(npf(q), npf(k), np.abs(npf(v)), causal=causal, attn_mask=m_np)
        bound = 2.0 ** -8 * (spv + 2 * np.abs(want)) * 1.01 + 2e-6
        assert np.all(np.abs(npf(ob) - want) <= bound)
    else:
        want = ref.attention_reference(npf(q), npf(k), npf(v), causal=causal, attn_mask=m_np,
                                       return_f32=True)
        assert_parity(ob, want, "key bytes")


PADDING_CASES = [
    # B, Hq, Hkv, Nq, Nk, D, bf16, per-row (packed bits) instead of key bytes
    (6, 14, 2, 1, 9000, 64, False, False),   # decode, splits + combine
    (5, 32, 8, 1, 4100, 128, True, False),   # bf16
    (4, 8, 2, 4, 3000, 128, False, True),    # 16 rows per unit, packed per-row words
    (3, 4, 4, 300, 1500, 64, False, False),  # small launch (row blocks of 32)
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,bf16,per_row", PADDING_CASES)
def test_padding_layouts_skip_hidden_tiles(device, B, Hq, Hkv, Nq, Nk, D, bf16, per_row):
    """The split-K kernel does not read K/V tiles that no query row of a
    workgroup sees (a padded batch's padding).  Contiguous padding hides
    whole 32-key tiles: right padding, left padding, a hole, a sequence with
    every key hidden (O = 0, LSE = -inf) and one that sees only its last key,
    one per batch entry; against the oracle incl. LSE."""
    print(f"[padding] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} bf16={bf16} per_row={per_row}",
          flush=True)
    dt = torch.bfloat16 if bf16 else torch.float16
    g = torch.Generator("cpu").manual_seed(Nk + B)
    q = torch.randn(B, Hq, Nq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, Nk, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, Nk, D, generator=g).to(dt)
    keys = torch.zeros(B, Nk, dtype=torch.bool)
    layouts = [(0, Nk // 3), (Nk - Nk // 5, Nk), (0, Nk)]  # right pad, left pad, full
    for b in range(B):
        kind = b % 6
        if kind < 3:
            lo, hi = layouts[kind]
            keys[b, lo:hi] = True
        elif kind == 3:  # a hole in the middle
            keys[b] = True
            keys[b, Nk // 4: Nk // 2] = False
        elif kind == 4:  # every key hidden
            pass
        else:  # only the last key
            keys[b, Nk - 1] = True
    m = keys[:, None, None, :]
    if per_row:
        m = m.expand(B, Hq, Nq, Nk).contiguous()
    o, lse = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                        return_lse=True, attn_mask=m.to(device))
    torch.cuda.synchronize()
    npf = lambda t: t.float().numpy()
    m_np = np.broadcast_to(m.numpy(), (B, Hq, Nq, Nk))
    got = o.float().cpu().numpy()
    assert np.isfinite(got).all()
    if bf16:
        want = ref.attention_f64(npf(q), npf(k), npf(v), attn_mask=m_np)
        spv = ref.attention_f64(npf(q), npf(k), np.abs(npf(v)), attn_mask=m_np)
        assert np.all(np.abs(got - want) <= 2.0 ** -8 * (spv + 2 * np.abs(want)) * 1.01 + 2e-6)
    else:
        want = ref.attention_reference(npf(q), npf(k), npf(v), attn_mask=m_np, return_f32=True)
        assert_parity(o, want, "padding")
    if B > 4:
        assert np.all(got[4] == 0)  # the sequence that sees no key
    wl = ref.attention_lse(npf(q), npf(k), attn_mask=m_np)
    gl = lse.cpu().numpy()
    fin = np.isfinite(wl)
    assert np.array_equal(np.isfinite(gl), fin)
    tol = float(np.log1p(2.0 ** -8)) + 1e-5 if bf16 else 1e-3
    np.testing.assert_allclose(gl[fin], wl[fin], atol=tol, rtol=0 if bf16 else 1e-4)


def _pack_ranges_lib():
    lib = ctypes.CDLL(LIB)
    f = lib.fa_sm75_pack_mask_ranges
    f.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p] * 3
    f.restype = ctypes.c_int
    return lib


@pytest.mark.parametrize("nk,sk", [(1, 1), (200, 1), (1500, 1), (2500, 1), (4100, 1), (8192, 1),
                                   (9001, 1), (300, 3)])
def test_pack_mask_ranges(device, nk, sk):
    """Each row's first visible key and one past the last ([nk, 0] for a row
    that sees none), bit 31 of the first set exactly when every key between
    them is visible, next to the same bits as fa_sm75_pack_mask, for rows of
    consecutive bytes and strided ones."""
    lib = _pack_ranges_lib()
    B, H, R = 2, 3, 5
    g = torch.Generator("cpu").manual_seed(nk)
    m = torch.zeros(B, H, R, nk * sk, dtype=torch.bool)
    for b in range(B):
        for h in range(H):
            for r in range(R):
                kind = (b * 15 + h * 5 + r) % 5
                if kind == 0:  # empty row
                    continue
                lo = int(torch.randint(0, nk, (1,), generator=g))
                hi = int(torch.randint(lo + 1, nk + 1, (1,), generator=g)) if kind != 3 else lo + 1
                row = torch.rand(nk, generator=g) < (1.0 if kind == 4 else 0.5)  # 4: an interval
                row[:lo] = False
                row[hi:] = False
                row[lo] = True
                row[hi - 1] = True
                m[b, h, r, ::sk] = row
    mv = m[..., ::sk]
    md = m.to(device)[..., ::sk]
    words = (nk + 63) // 64
    out = torch.full((B, H, R, words), -1, dtype=torch.int64, device=device)
    ranges = torch.full((B, H, R, 2), -7, dtype=torch.int32, device=device)
    st = md.stride()
    assert lib.fa_sm75_pack_mask_ranges(md.data_ptr(), B, H, R, nk, st[0], st[1], st[2], st[3],
                                        out.data_ptr(), ranges.data_ptr(),
                                        torch.cuda.current_stream().cuda_stream) == 0
    torch.cuda.synchronize()
    mn = mv.numpy()
    padded = np.zeros((B, H, R, words * 64), dtype=np.uint8)
    padded[..., :nk] = mn
    want = np.packbits(padded.reshape(B, H, R, words, 64), axis=-1, bitorder="little")
    assert np.array_equal(out.cpu().numpy().view(np.uint64), want.view(np.uint64).reshape(out.shape))
    got = ranges.cpu().numpy()
    for b in range(B):
        for h in range(H):
            for r in range(R):
                idx = np.nonzero(mn[b, h, r])[0]
                exp = (idx[0], idx[-1] + 1) if idx.size else (nk, 0)
                dense = idx.size > 0 and idx[-1] + 1 - idx[0] == idx.size
                first = int(got[b, h, r, 0])
                assert (first & 0x7FFFFFFF, int(got[b, h, r, 1])) == exp, (b, h, r, first, exp)
                assert (first < 0) == dense, (b, h, r, first, dense)


RANGE_CASES = [
    # B, Hq, Hkv, Nq, Nk, D, bf16, mask kind, policy
    (2, 4, 2, 1000, 1000, 128, False, "causal+pad", 0),   # transformers' padded prefill
    (3, 8, 2, 700, 700, 64, True, "causal+pad", 0),
    (2, 4, 4, 300, 900, 64, False, "causal+pad", 0),       # Nq < Nk (chunked prefill with cache)
    (2, 16, 4, 2048, 2048, 128, False, "causal+pad", 3),   # dynamic schedule: several items per WG
    (2, 4, 2, 513, 513, 128, False, "per-head", 0),        # random per-head rows
    # rows that see exactly an interval (bit 31 of the first entry): a sliding window of its
    # own width per head, and causal padding with holes punched into a few rows, so some
    # waves mix interval rows with others and must read their mask words
    (2, 4, 2, 900, 900, 64, False, "window", 0),
    (1, 8, 2, 1100, 1100, 128, False, "holes", 0),
    (2, 4, 4, 700, 700, 128, True, "holes", 3),
    # 256-row workgroups (policy WIDE), also bitwise against the 128-row kernel
    (2, 4, 2, 1000, 1000, 128, False, "causal+pad", 2),
    (3, 8, 2, 700, 700, 64, True, "causal+pad", 2),
    (2, 4, 2, 513, 513, 128, False, "per-head", 2),
    (2, 4, 2, 900, 900, 64, False, "window", 2),
    (1, 8, 2, 1100, 1100, 128, False, "holes", 2),
]


def _range_mask(kind, B, Hq, Nq, Nk, g):
    if kind == "per-head":
        return torch.rand(B, Hq, Nq, Nk, generator=g) < 0.3
    if kind == "window":  # query i sees keys (i - w_h, i], w_h per head
        i = torch.arange(Nq)[:, None]
        j = torch.arange(Nk)[None, :]
        m = torch.zeros(B, Hq, Nq, Nk, dtype=torch.bool)
        for h in range(Hq):
            w = [37, 150, 400, Nk][h % 4]
            m[:, h] = (j <= i) & (j > i - w)
        return m
    # causal (bottom-right for Nq < Nk) and left padding of B different lengths
    i = torch.arange(Nq)[:, None] + (Nk - Nq)
    j = torch.arange(Nk)[None, :]
    m = (j <= i)[None, None].expand(B, 1, Nq, Nk).clone()
    for b in range(B):
        pad = (b * Nk) // (2 * B)
        m[b, :, :, :pad] = False
    if kind == "holes":  # a hidden key inside the interval of every 40th row
        for r in range(5, Nq, 40):
            m[:, :, r, r // 2] = False
    return m


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,bf16,kind,policy", RANGE_CASES)
def test_mask_ranges_skip_tiles(device, B, Hq, Hkv, Nq, Nk, D, bf16, kind, policy):
    """Through the C ABI: the same packed mask with and without mask_ranges
    gives the same O and LSE bit for bit (the skipped tiles hide every key
    from every row of their block), and the result meets the oracle's bar."""
    from capi_types import Params
    print(f"[ranges] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} bf16={bf16} {kind} "
          f"policy={policy}", flush=True)
    lib = _pack_ranges_lib()
    lib.fa_sm75_forward.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.restype = ctypes.c_int64
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    dt = torch.bfloat16 if bf16 else torch.float16
    g = torch.Generator("cpu").manual_seed(Nq * 7 + Nk)
    q = torch.randn(B, Hq, Nq, D, generator=g).to(dt).to(device)
    k = torch.randn(B, Hkv, Nk, D, generator=g).to(dt).to(device)
    v = torch.randn(B, Hkv, Nk, D, generator=g).to(dt).to(device)
    m = _range_mask(kind, B, Hq, Nq, Nk, g)
    md = m.to(device)
    Hm = m.shape[1]
    words = (Nk + 63) // 64
    bits = torch.empty(B, Hm, Nq, words, dtype=torch.int64, device=device)
    ranges = torch.empty(B, Hm, Nq, 2, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    st = md.stride()
    assert lib.fa_sm75_pack_mask_ranges(md.data_ptr(), B, Hm, Nq, Nk, st[0], st[1], st[2], st[3],
                                        bits.data_ptr(), ranges.data_ptr(), stream) == 0

    def run(with_ranges):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((B, Hq, Nq), float("nan"), device=device)
        p = Params()
        p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
        p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = B, Hq, Hkv, Nq, D
        p.seq_len_kv = Nk
        lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
        p.scale, p.dtype, p.stream = D ** -0.5, 1 if bf16 else 0, stream
        p.mask_bits = bits.data_ptr()
        p.mask_stride_b, p.mask_stride_h, p.mask_stride_q = Hm * Nq * words, (Nq * words if Hm > 1 else 0), words
        if with_ranges:
            p.mask_ranges = ranges.data_ptr()
            p.mask_ranges_stride_b, p.mask_ranges_stride_h, p.mask_ranges_stride_q = Hm * Nq, (Nq if Hm > 1 else 0), 1
        n = lib.fa_sm75_workspace_size(ctypes.byref(p))
        ws = torch.empty(max(n, 16), dtype=torch.uint8, device=device)
        p.workspace, p.workspace_bytes = ws.data_ptr(), n
        assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
        torch.cuda.synchronize()
        return o, lse

    assert lib.fa_sm75_set_kernel_policy(policy) == 0
    try:
        o1, l1 = run(True)
        o0, l0 = run(False)
        if policy == 2:
            assert lib.fa_sm75_set_kernel_policy(1) == 0
            on, ln = run(True)
    finally:
        lib.fa_sm75_set_kernel_policy(0)
    assert torch.equal(o1, o0) and torch.equal(l1, l0)
    if policy == 2:
        assert torch.equal(o1, on) and torch.equal(l1, ln)
    npf = lambda t: t.float().cpu().numpy()
    mn = np.broadcast_to(m.numpy(), (B, Hq, Nq, Nk))
    if bf16:
        want = ref.attention_f64(npf(q), npf(k), npf(v), attn_mask=mn)
        spv = ref.attention_f64(npf(q), npf(k), np.abs(npf(v)), attn_mask=mn)
        assert np.all(np.abs(npf(o1) - want) <= 2.0 ** -8 * (spv + 2 * np.abs(want)) * 1.01 + 2e-6)
    else:
        want = ref.attention_reference(npf(q), npf(k), npf(v), attn_mask=mn, return_f32=True)
        assert_parity(o1, want, "ranges")
