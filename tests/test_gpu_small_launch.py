"""The small-launch path on the GPU: launches whose 128-row prefill grid would
hold at most 64 workgroups (BASELINE C1: one head of 512 rows, 4 workgroups)
run on the split-K kernel with the query rows in blocks of 32, each block's
keys spread over the four waves of a workgroup (64 key tiles of 32 or fewer)
or over several workgroups and the combine kernel (more tiles).

Parity bar as everywhere: |O - O_ref| <= 2e-3 + 1e-2 |O_ref| and max-abs <=
2e-3 against the numpy oracle (fp32, reference math order) on the same seeded
inputs; LSE against the float64 closed form.  Each case is also compared with
the 128-row prefill kernel (policy NARROW) on the same inputs.
"""
import ctypes

import numpy as np
import pytest
import torch

from capi_types import LIB, Params
from flash_attention_sm75 import flash_attention_forward, flash_attention_forward_ex
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
CODE = {False: 0, True: 1, "top_left": 1, "bottom_right": 2}


def seeded(shape, seed, std=1.0, dtype=torch.float16):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).to(dtype)


def npf(t):
    return t.float().numpy()


def parity(out, expect, label, atol=ATOL, rtol=RTOL, max_abs=ATOL):
    out = out.detach().float().cpu().numpy()
    res = ref.check_correctness(out, expect, name=label, atol=atol, rtol=rtol)
    print(f"  {label}: max_abs={res['max_abs_err']:.3e}", flush=True)
    assert res["allclose"], res
    if max_abs is not None:
        assert res["max_abs_err"] <= max_abs, res


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    lib.fa_sm75_workspace_size.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.restype = ctypes.c_int64
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    return lib


def workspace_bytes(lib, B, Hq, Hkv, Nq, Nk, D, code):
    p = Params()
    p.q = p.k = p.v = p.o = 0x10000
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.seq_len_kv, p.head_dim = B, Hq, Hkv, Nq, Nk, D
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.scale, p.causal = D ** -0.5, code
    return lib.fa_sm75_workspace_size(ctypes.byref(p))


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal; (items = B*Hq*ceil(Nq/128) <= 64)
    (1, 1, 1, 512, 512, 64, False),           # C1
    (1, 1, 1, 512, 512, 128, True),
    (1, 8, 8, 512, 512, 64, False),
    (1, 4, 4, 1000, 1000, 64, True),          # tail rows and keys
    (1, 4, 2, 700, 700, 128, True),           # GQA: row blocks span two query heads
    (2, 6, 3, 333, 333, 64, False),
    (1, 2, 1, 200, 900, 64, "bottom_right"),  # Nq < Nk, bottom-right
    (1, 2, 2, 300, 120, 128, "top_left"),     # Nq > Nk: rows past the keys
    (1, 2, 2, 300, 120, 64, "bottom_right"),  # rows that see no key
    (1, 1, 1, 4096, 4096, 128, True),         # 128 key tiles: several splits + combine
    (1, 2, 1, 3000, 3000, 64, False),         # 94 tiles: several splits
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", CASES)
def test_small_launch_matches_oracle(device, lib, B, Hq, Hkv, Nq, Nk, D, causal):
    print(f"[small] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal}", flush=True)
    assert B * Hq * ((Nq + 127) // 128) <= 64
    code = CODE[causal]
    q, k, v = seeded((B, Hq, Nq, D), 1), seeded((B, Hkv, Nk, D), 2), seeded((B, Hkv, Nk, D), 3)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    o, lse = flash_attention_forward_ex(qd, kd, vd, causal=causal, return_lse=True)
    lib.fa_sm75_set_kernel_policy(1)  # the 128-row prefill kernel on the same call
    try:
        o_pre, lse_pre = flash_attention_forward_ex(qd, kd, vd, causal=causal, return_lse=True)
    finally:
        lib.fa_sm75_set_kernel_policy(0)
    torch.cuda.synchronize()
    tiles = (Nk + 31) // 32
    print(f"  workspace {workspace_bytes(lib, B, Hq, Hkv, Nq, Nk, D, code)} bytes, {tiles} key "
          f"tiles", flush=True)
    expect = ref.attention_reference_chunked(npf(q), npf(k), npf(v), causal=code, return_f32=True)
    parity(o, expect, "small-launch path")
    parity(o_pre, expect, "prefill kernel")
    want = ref.attention_lse(npf(q), npf(k), causal=code)
    got = lse.cpu().numpy()
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    np.testing.assert_allclose(got[fin], want[fin], atol=2e-4, rtol=1e-5)
    torch.testing.assert_close(lse, lse_pre, atol=1e-4, rtol=1e-5)


def test_small_launch_workspace_rule(lib):
    """Up to 64 key tiles of 32: one split, no workspace; more: splits."""
    assert workspace_bytes(lib, 1, 1, 1, 512, 512, 64, 0) == 0
    assert workspace_bytes(lib, 1, 8, 8, 512, 512, 64, 0) == 0
    assert workspace_bytes(lib, 1, 1, 1, 4096, 4096, 128, 1) > 0
    assert workspace_bytes(lib, 1, 2, 1, 3000, 3000, 64, 0) > 0


@pytest.mark.parametrize("mshape", ["b11k", "bhqk"])
def test_small_launch_boolean_mask(device, mshape):
    B, Hq, Hkv, N, D = 2, 4, 2, 400, 64
    print(f"[small mask] {mshape}", flush=True)
    g = torch.Generator("cpu").manual_seed(21)
    shape = (B, 1, 1, N) if mshape == "b11k" else (B, Hq, N, N)
    mask = torch.rand(*shape, generator=g) < 0.7
    if mshape == "b11k":
        mask[1, ..., N - 50:] = False  # batch 1 right-padded
    q, k, v = seeded((B, Hq, N, D), 4), seeded((B, Hkv, N, D), 5), seeded((B, Hkv, N, D), 6)
    o = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                   attn_mask=mask.to(device))
    torch.cuda.synchronize()
    expect = ref.attention_reference_chunked(npf(q), npf(k), npf(v), return_f32=True,
                                             attn_mask=mask.numpy())
    parity(o, expect, f"mask {mshape}")


def test_small_launch_bf16(device):
    B, Hq, Hkv, N, D = 1, 4, 1, 600, 128
    q, k, v = (seeded(s, i, dtype=torch.bfloat16) for i, s in
               enumerate(((B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D)), 7))
    o = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device), causal=True)
    torch.cuda.synchronize()
    expect = ref.attention_reference_chunked(npf(q), npf(k), npf(v), causal=1, return_f32=True)
    # the bfloat16 bar (8 fewer output mantissa bits than binary16)
    parity(o, expect, "bf16", atol=4e-3, rtol=1.6e-2, max_abs=None)


def test_reference_launcher_without_workspace(device):
    """The reference-named op path (C1 through flash_attention_forward): the
    same bytes as the C ABI call with a workspace of the size it asks for."""
    q, k, v = (seeded((1, 1, 512, 64), s).to(device) for s in (30, 31, 32))
    a = flash_attention_forward(q, k, v)
    b = flash_attention_forward_ex(q, k, v)
    torch.cuda.synchronize()
    assert torch.equal(a, b)
