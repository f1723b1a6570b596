"""Calls straight through the C ABI (ctypes) on device buffers (needs a GPU).

Checks that the stream-ordered entry point and the reference-signature
launchers produce the same bytes as the binding, and that fa_sm75_forward
honours non-contiguous strides.
"""
import ctypes

import pytest
import torch

import flash_attn_sm75_cuda as _C

from capi_types import LIB, Params

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_forward.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_forward.restype = ctypes.c_int
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    sig = [ctypes.c_void_p] * 4 + [ctypes.c_int] * 4 + [ctypes.c_float, ctypes.c_bool]
    for n in ("launch_flash_attention_forward", "launch_flash_attention_forward_scalar",
              "launch_flash_attention_forward_wmma_qk"):
        getattr(lib, n).argtypes = sig
        getattr(lib, n).restype = None
    lib.launch_naive_attention.argtypes = sig + [ctypes.c_void_p]
    lib.launch_naive_attention.restype = None
    return lib


def inputs(B, H, Hkv, N, D, seed, device):
    g = torch.Generator("cpu").manual_seed(seed)
    return [torch.randn(B, h, N, D, generator=g).half().to(device) for h in (H, Hkv, Hkv)]


@pytest.mark.parametrize("D,causal", [(64, False), (128, True)])
def test_stream_entry_matches_binding(device, lib, D, causal):
    q, k, v = inputs(2, 8, 2, 333, D, 1, device)
    o = torch.empty_like(q)
    lse = torch.empty(2, 8, 333, dtype=torch.float32, device=device)
    p = Params()
    p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = 2, 8, 2, 333, D
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.scale, p.causal = 0.1, int(causal)
    p.stream = torch.cuda.current_stream().cuda_stream
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
    ref_o, ref_lse = _C.flash_attention_forward_lse(q, k, v, causal, 0.1)
    torch.cuda.synchronize()
    assert torch.equal(o, ref_o)
    assert torch.equal(lse, ref_lse)


def test_strided_views(device, lib):
    """Q/K/V/O as [B, N, H, D] buffers viewed as [B, H, N, D] (row stride H*D)."""
    B, H, Hkv, N, D = 1, 4, 2, 150, 64
    g = torch.Generator("cpu").manual_seed(2)
    qb = torch.randn(B, N, H, D, generator=g).half().to(device)
    kb = torch.randn(B, N, Hkv, D, generator=g).half().to(device)
    vb = torch.randn(B, N, Hkv, D, generator=g).half().to(device)
    ob = torch.zeros(B, N, H, D, dtype=torch.float16, device=device)
    p = Params()
    p.q, p.k, p.v, p.o = qb.data_ptr(), kb.data_ptr(), vb.data_ptr(), ob.data_ptr()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = B, H, Hkv, N, D
    p.q_stride_b, p.q_stride_h, p.q_stride_n = N * H * D, D, H * D
    p.o_stride_b, p.o_stride_h, p.o_stride_n = N * H * D, D, H * D
    p.k_stride_b, p.k_stride_h, p.k_stride_n = N * Hkv * D, D, Hkv * D
    p.v_stride_b, p.v_stride_h, p.v_stride_n = N * Hkv * D, D, Hkv * D
    p.scale, p.causal = 0.125, 1
    p.stream = torch.cuda.current_stream().cuda_stream
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
    expect = _C.flash_attention_forward(qb.transpose(1, 2).contiguous(), kb.transpose(1, 2).contiguous(),
                                        vb.transpose(1, 2).contiguous(), True, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(ob.transpose(1, 2), expect)


def test_reference_launchers(device, lib):
    torch.cuda.synchronize()
    q, k, v = inputs(1, 4, 4, 200, 64, 3, device)
    main = _C.flash_attention_forward(q, k, v, True, 0.125)
    torch.cuda.synchronize()
    for n in ("launch_flash_attention_forward", "launch_flash_attention_forward_scalar",
              "launch_flash_attention_forward_wmma_qk"):
        o = torch.zeros_like(q)
        torch.cuda.synchronize()
        getattr(lib, n)(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), 1, 4, 200, 64,
                        0.125, True)
        assert torch.equal(o, main), n
    ws = torch.empty(4 * 200 * 200, dtype=torch.float32, device=device)
    o = torch.zeros_like(q)
    lib.launch_naive_attention(q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), 1, 4, 200,
                               64, 0.125, True, ws.data_ptr())
    assert (o.float() - main.float()).abs().max().item() < 4e-3


def test_legacy_launcher_rejects_bad_head_dim(device, lib, capfd):
    q = torch.full((1, 1, 16, 96), 7.0, dtype=torch.float16, device=device)
    o = torch.full_like(q, 3.0)
    torch.cuda.synchronize()
    lib.launch_flash_attention_forward(q.data_ptr(), q.data_ptr(), q.data_ptr(), o.data_ptr(),
                                       1, 1, 16, 96, 0.1, False)
    err = capfd.readouterr().err
    assert "head_dim=64 or 128" in err
    assert torch.all(o == 3.0)  # untouched, as the reference launcher leaves it


@pytest.mark.parametrize("causal", [0, 1, 2])
def test_separate_kv_length_matches_binding(device, lib, causal):
    """fa_sm75_forward with seq_len_kv != seq_len gives the binding's bytes."""
    B, H, Hkv, Nq, Nk, D = 2, 4, 2, 50, 211, 64
    g = torch.Generator("cpu").manual_seed(30 + causal)
    q = torch.randn(B, H, Nq, D, generator=g).half().to(device)
    k = torch.randn(B, Hkv, Nk, D, generator=g).half().to(device)
    v = torch.randn(B, Hkv, Nk, D, generator=g).half().to(device)
    o = torch.empty_like(q)
    p = Params()
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = B, H, Hkv, Nq, D
    p.seq_len_kv = Nk
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.scale, p.causal = 0.125, causal
    p.stream = torch.cuda.current_stream().cuda_stream
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
    expect = _C.flash_attention_forward_ex(q, k, v, causal, 0.125, False)[0]
    torch.cuda.synchronize()
    assert torch.equal(o, expect)


def test_decode_mask_span_over_2gib(device, lib):
    """A split-K-eligible call (group * Nq <= 32) whose mask strides span more
    than the split-K kernel's 32-bit mask window: head 1's words sit 2 GiB
    past head 0's.  The call must run on the prefill kernel (64-bit mask
    addresses) and give the same result as the packed, contiguous mask."""
    from flash_attention_sm75 import flash_attention_forward_ex

    B, Hq, Hkv, Nq, Nk, D = 1, 2, 1, 1, 1000, 64
    words = (Nk + 63) // 64
    msh = (1 << 28) + 64  # words: 2 GiB + 512 bytes between the heads' rows
    print(f"[decode mask span] head stride {msh * 8} bytes", flush=True)
    g = torch.Generator("cpu").manual_seed(70)
    q, k, v = (torch.randn(B, h, n, D, generator=g).half().to(device)
               for h, n in ((Hq, Nq), (Hkv, Nk), (Hkv, Nk)))
    vis = torch.rand(B, Hq, Nq, Nk, generator=g) < 0.6
    packed = torch.zeros(Hq, words, dtype=torch.int64)
    for h in range(Hq):
        bits = vis[0, h, 0].tolist() + [False] * (64 * words - Nk)
        for w in range(words):
            word = sum(1 << i for i in range(64) if bits[64 * w + i])
            packed[h, w] = word - (1 << 64) if word >= (1 << 63) else word
    big = torch.zeros(msh * (Hq - 1) + words, dtype=torch.int64, device=device)
    for h in range(Hq):
        big[h * msh:h * msh + words] = packed[h].to(device)
    o = torch.empty_like(q)
    p = Params()
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.seq_len_kv, p.head_dim = B, Hq, Hkv, Nq, Nk, D
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.scale, p.causal = 0.125, 0
    p.mask_bits = big.data_ptr()
    p.mask_stride_b, p.mask_stride_h, p.mask_stride_q = 0, msh, words
    p.stream = torch.cuda.current_stream().cuda_stream
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
    want = flash_attention_forward_ex(q, k, v, scale=0.125, attn_mask=vis.to(device))
    torch.cuda.synchronize()
    del big
    torch.testing.assert_close(o, want, atol=2e-3, rtol=1e-2)
