"""The split-K path (few query rows per K/V head: KV-cache decode) on the GPU.

fa_sm75_forward takes it when heads_q / heads_kv * seq_len <= 32.  Parity bar
as everywhere: |O - O_ref| <= 2e-3 + 1e-2 |O_ref| against the numpy oracle
on the same seeded inputs; LSE against the float64 closed form.  The path is
also checked against the 128-row prefill kernel (forced through the kernel
policy) and against itself with and without a workspace (one split vs many).
"""
import ctypes

import numpy as np
import pytest
import torch

from capi_types import LIB, Params
from flash_attention_sm75 import flash_attention_forward_ex
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2


def seeded(shape, seed, std=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    return (torch.randn(*shape, generator=g) * std).half()


def assert_parity(out, expect, label):
    out = out.detach().float().cpu().numpy()
    res = ref.check_correctness(out, expect, name=label, atol=ATOL, rtol=RTOL)
    print(f"  {label}: max_abs={res['max_abs_err']:.3e}", flush=True)
    assert res["allclose"], res


def check_lse(lse, q, k, code):
    want = ref.attention_lse(q.numpy(), k.numpy(), causal=code)
    got = lse.cpu().numpy()
    fin = np.isfinite(want)
    assert np.array_equal(np.isfinite(got), fin)
    np.testing.assert_allclose(got[fin], want[fin], atol=1e-3, rtol=1e-4)


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal
    (4, 32, 8, 1, 8192, 128, False),      # Llama-style decode step
    (2, 14, 2, 1, 3000, 64, False),       # Qwen2-0.5B heads (group 7)
    (1, 64, 8, 4, 5000, 128, "bottom_right"),  # 4 draft tokens: 32 rows
    (3, 8, 8, 2, 77, 64, "top_left"),
    (1, 32, 1, 1, 60000, 128, False),     # long context, one KV head (MQA)
    (1, 7, 1, 1, 50000, 64, "bottom_right"),  # 195 splits: the wide combine at d64
    (2, 4, 2, 1, 1, 128, False),          # a single key
    (2, 4, 2, 3, 31, 64, "bottom_right"),
    (2, 4, 2, 3, 33, 128, False),
    (1, 16, 2, 2, 4099, 128, "top_left"),  # top-left decode sees keys 0..1
    (2, 8, 4, 16, 16, 64, True),          # small square causal (also routed here)
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", CASES)
def test_decode_matches_oracle(device, B, Hq, Hkv, Nq, Nk, D, causal):
    print(f"[case] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal}", flush=True)
    q = seeded((B, Hq, Nq, D), 1)
    k = seeded((B, Hkv, Nk, D), 2)
    v = seeded((B, Hkv, Nk, D), 3)
    code = {False: 0, True: 1, "top_left": 1, "bottom_right": 2}[causal]
    o, lse = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                        causal=causal, return_lse=True)
    torch.cuda.synchronize()
    expect = ref.attention_reference_chunked(q.numpy(), k.numpy(), v.numpy(), causal=code,
                                             return_f32=True)
    assert_parity(o, expect, f"B{B} H{Hq}/{Hkv} Nq{Nq} Nk{Nk} D{D} c={causal}")
    check_lse(lse, q, k, code)


def test_decode_large_keys_in_k(device):
    """C5-style stress: K rows x4 on 5% of keys, scores far apart."""
    B, Hq, Hkv, Nk, D = 2, 16, 2, 20000, 128
    g = torch.Generator("cpu").manual_seed(9)
    q = (torch.randn(B, Hq, 1, D, generator=g) * 0.5).half()
    k = torch.randn(B, Hkv, Nk, D, generator=g) * 0.5
    boost = torch.rand(B, Hkv, Nk, 1, generator=g) < 0.05
    k = torch.where(boost, k * 4, k).half()
    v = (torch.randn(B, Hkv, Nk, D, generator=g) * 0.5).half()
    o = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device))
    torch.cuda.synchronize()
    expect = ref.attention_reference(q.numpy(), k.numpy(), v.numpy(), return_f32=True)
    assert_parity(o, expect, "decode K x4")


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_forward.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_forward.restype = ctypes.c_int
    lib.fa_sm75_workspace_size.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.restype = ctypes.c_int64
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    return lib


def capi_forward(lib, q, k, v, causal, workspace=None, policy=0):
    B, Hq, Nq, D = q.shape
    o = torch.full_like(q, float("nan"))
    lse = torch.empty(B, Hq, Nq, dtype=torch.float32, device=q.device)
    p = Params()
    p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = B, Hq, k.shape[1], Nq, D
    p.seq_len_kv = k.shape[2]
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.scale, p.causal = D ** -0.5, causal
    p.stream = torch.cuda.current_stream().cuda_stream
    if workspace is not None:
        p.workspace, p.workspace_bytes = workspace.data_ptr(), workspace.numel()
    assert lib.fa_sm75_set_kernel_policy(policy) == 0
    try:
        assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
    finally:
        lib.fa_sm75_set_kernel_policy(0)
    return o, lse, p


@pytest.mark.parametrize("Nq,causal", [(1, 0), (4, 2)])
def test_workspace_and_policies_agree(device, lib, Nq, causal):
    """Many splits (workspace), one split (no workspace) and the prefill
    kernel (policy NARROW) all meet the bar against the oracle and agree."""
    B, Hq, Hkv, Nk, D = 2, 32, 4, 7777, 128
    q = seeded((B, Hq, Nq, D), 11).to(device)
    k = seeded((B, Hkv, Nk, D), 12).to(device)
    v = seeded((B, Hkv, Nk, D), 13).to(device)
    p0 = capi_forward(lib, q, k, v, causal)[2]
    ws_bytes = lib.fa_sm75_workspace_size(ctypes.byref(p0))
    assert ws_bytes > 0
    ws = torch.empty(ws_bytes, dtype=torch.uint8, device=device)
    o_split, lse_split, _ = capi_forward(lib, q, k, v, causal, workspace=ws)
    o_one, lse_one, _ = capi_forward(lib, q, k, v, causal)
    o_pre, lse_pre, _ = capi_forward(lib, q, k, v, causal, policy=1)
    torch.cuda.synchronize()
    expect = ref.attention_reference_chunked(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(),
                                             causal=causal, return_f32=True)
    for o, name in ((o_split, "splits"), (o_one, "one split"), (o_pre, "prefill kernel")):
        assert_parity(o, expect, name)
    for lse in (lse_split, lse_one):
        torch.testing.assert_close(lse, lse_pre, atol=1e-4, rtol=1e-5)


def test_workspace_reuse_second_call_smaller(device, lib):
    """The same workspace serves a second, smaller call (stale partials of the
    first call must not leak into the second)."""
    q = seeded((2, 16, 1, 64), 14).to(device)
    k = seeded((2, 2, 9000, 64), 15).to(device)
    v = seeded((2, 2, 9000, 64), 16).to(device)
    p0 = capi_forward(lib, q, k, v, 0)[2]
    ws = torch.empty(lib.fa_sm75_workspace_size(ctypes.byref(p0)), dtype=torch.uint8, device=device)
    o1 = capi_forward(lib, q, k, v, 0, workspace=ws)[0]
    k2, v2 = k[:, :, :3000].contiguous(), v[:, :, :3000].contiguous()
    o2 = capi_forward(lib, q[:1], k2[:1], v2[:1], 0, workspace=ws)[0]
    torch.cuda.synchronize()
    e1 = ref.attention_reference(q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy(), return_f32=True)
    e2 = ref.attention_reference(q[:1].cpu().numpy(), k2[:1].cpu().numpy(), v2[:1].cpu().numpy(),
                                 return_f32=True)
    assert_parity(o1, e1, "first call")
    assert_parity(o2, e2, "second call")
