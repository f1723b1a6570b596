"""Dynamic (XCD-balanced) schedule of the fused kernel, through the C ABI.

With a workspace of fa_sm75_workspace_size() bytes and more query blocks
than resident workgroups, fa_sm75_forward runs the persistent kernel that
claims query blocks from per-XCD queues.  Every block is computed by the
same code as in the static one-workgroup-per-block schedule, so O and LSE
must be bitwise identical to the static run; one case is also held to the
oracle.  Covered: GQA causal (8 queues), units not divisible by 8 (one
queue), bottom-right alignment with blocks that see no key, an explicit
mask, a garbage-filled and reused workspace (smaller second call), and two
streams with their own workspaces at once.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

import flash_attn_sm75_cuda as _C
from oracle import attention_ref as ref

from capi_types import LIB, Params

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_forward.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_forward.restype = ctypes.c_int
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    lib.fa_sm75_workspace_size.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.restype = ctypes.c_int64
    return lib


def seeded(shape, seed, device):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g).half().to(device)


@pytest.fixture(autouse=True)
def restore_policy(lib):
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    yield
    lib.fa_sm75_set_kernel_policy(0)


def run(lib, q, k, v, causal, workspace=None, mask=None, stream=None):
    """One fa_sm75_forward call; returns (O, LSE).  With a workspace the
    dynamic schedule is forced (policy DYNAMIC), without one the static
    schedule runs (policy NARROW)."""
    B, Hq, N, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    s = stream if stream is not None else torch.cuda.current_stream()
    # The NaN fills run on the launch stream, so they are ordered before the
    # kernel that overwrites them.
    with torch.cuda.stream(s):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((B, Hq, N), float("nan"), dtype=torch.float32, device=q.device)
    p = Params()
    p.q, p.k, p.v, p.o, p.lse = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(), lse.data_ptr()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = B, Hq, Hkv, N, D
    p.seq_len_kv = Nk
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.scale, p.causal = 1.0 / math.sqrt(D), causal
    p.stream = s.cuda_stream
    if workspace is not None:
        p.workspace, p.workspace_bytes = workspace.data_ptr(), workspace.numel()
    if mask is not None:
        bits, (sb, sh, sq) = mask
        p.mask_bits = bits.data_ptr()
        p.mask_stride_b, p.mask_stride_h, p.mask_stride_q = sb, sh, sq
    assert lib.fa_sm75_set_kernel_policy(3 if workspace is not None else 1) == 0
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
    return o, lse


def workspace_for(lib, q, k, causal, device, fill=0xA5):
    p = Params()
    # validated like a call (non-null, aligned pointers); nothing is launched
    p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), k.data_ptr(), q.data_ptr()
    B, Hq, N, D = q.shape
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = B, Hq, k.shape[1], N, D
    p.seq_len_kv = k.shape[2]
    p.scale, p.causal = 1.0 / math.sqrt(D), causal
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    assert lib.fa_sm75_set_kernel_policy(3) == 0
    n = lib.fa_sm75_workspace_size(ctypes.byref(p))
    assert n >= 2048, n
    # The contents on entry must not matter.
    return torch.full((n,), fill, dtype=torch.uint8, device=device)


def resident(device):
    return 2 * torch.cuda.get_device_properties(device).multi_processor_count


CASES = [
    # (B, Hq, Hkv, N, Nk, D, causal): query blocks > resident workgroups
    (2, 32, 8, 1100, 1100, 128, 1),   # GQA 4:1, 8 queues (one per XCD)
    (1, 24, 3, 3000, 3000, 64, 0),    # 3 units: one queue, full attention
    (1, 32, 8, 3000, 1000, 128, 2),   # bottom-right: the first blocks see no key
    (3, 40, 8, 700, 900, 64, 1),      # top-left, Nq != Nk, 8 queues
]


@pytest.mark.parametrize("B,Hq,Hkv,N,Nk,D,causal", CASES)
def test_dynamic_matches_static(device, lib, B, Hq, Hkv, N, Nk, D, causal):
    assert B * Hq * math.ceil(N / 128) > resident(device)
    q = seeded((B, Hq, N, D), 1, device)
    k = seeded((B, Hkv, Nk, D), 2, device)
    v = seeded((B, Hkv, Nk, D), 3, device)
    ws = workspace_for(lib, q, k, causal, device)
    o_s, lse_s = run(lib, q, k, v, causal)
    o_d, lse_d = run(lib, q, k, v, causal, workspace=ws)
    o_d2, lse_d2 = run(lib, q, k, v, causal, workspace=ws)  # reused workspace
    torch.cuda.synchronize()
    assert not torch.isnan(o_d).any()
    assert torch.equal(o_d, o_s) and torch.equal(o_d2, o_s)
    assert torch.equal(lse_d, lse_s) and torch.equal(lse_d2, lse_s)


def test_dynamic_against_oracle(device, lib):
    """Independent check of one dynamic run: sampled heads against the oracle."""
    B, Hq, Hkv, N, D = 1, 40, 8, 1700, 128
    q, k, v = (seeded((B, h, N, D), s, device) for s, h in ((4, Hq), (5, Hkv), (6, Hkv)))
    ws = workspace_for(lib, q, k, 1, device)
    o, lse = run(lib, q, k, v, 1, workspace=ws)
    torch.cuda.synchronize()
    heads = [0, 13, 39]
    qn, kn, vn = q.cpu().numpy(), k.cpu().numpy(), v.cpu().numpy()
    group = Hq // Hkv
    for h in heads:
        kv = h // group
        exp = ref.attention_reference(qn[:, h:h + 1], kn[:, kv:kv + 1], vn[:, kv:kv + 1],
                                      causal=True, return_f32=True)
        res = ref.check_correctness(o[:, h:h + 1].float().cpu().numpy(), exp, atol=2e-3, rtol=1e-2)
        assert res["allclose"], (h, res)
        exp_lse = ref.attention_lse(qn[:, h:h + 1], kn[:, kv:kv + 1], causal=True)
        np.testing.assert_allclose(lse[:, h:h + 1].cpu().numpy(), exp_lse, atol=2e-4, rtol=1e-5)


def test_dynamic_with_mask(device, lib):
    """Masked calls take the 4-wave kernel, so the dynamic schedule too."""
    B, Hq, Hkv, N, D = 2, 32, 8, 1100, 64
    q, k, v = (seeded((B, h, N, D), s, device) for s, h in ((7, Hq), (8, Hkv), (9, Hkv)))
    g = torch.Generator("cpu").manual_seed(10)
    keep = (torch.rand(B, 1, N, N, generator=g) > 0.2).to(device)
    pack = lib.fa_sm75_pack_mask
    pack.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p, ctypes.c_void_p]
    pack.restype = ctypes.c_int
    words = (N + 63) // 64
    bits = torch.empty(B, 1, N, words, dtype=torch.int64, device=device)
    st = keep.stride()
    assert pack(keep.data_ptr(), B, 1, N, N, st[0], st[1], st[2], st[3], bits.data_ptr(),
                torch.cuda.current_stream().cuda_stream) == 0
    mask = (bits, (N * words, 0, words))  # broadcast over the heads
    ws = workspace_for(lib, q, k, 0, device)
    o_s, lse_s = run(lib, q, k, v, 0, mask=mask)
    o_d, lse_d = run(lib, q, k, v, 0, workspace=ws, mask=mask)
    torch.cuda.synchronize()
    assert torch.equal(o_d, o_s) and torch.equal(lse_d, lse_s)


def test_workspace_reuse_second_call_smaller(device, lib):
    """The workspace keeps the previous call's counters; the next call
    (smaller, on the same stream) must start from cleared queues."""
    ws = None
    for (B, N) in ((2, 2000), (1, 2100)):
        q = seeded((B, 32, N, 128), 11 + N, device)
        k = seeded((B, 8, N, 128), 12 + N, device)
        v = seeded((B, 8, N, 128), 13 + N, device)
        if ws is None:
            ws = workspace_for(lib, q, k, 1, device)
        o_s, lse_s = run(lib, q, k, v, 1)
        o_d, lse_d = run(lib, q, k, v, 1, workspace=ws)
        torch.cuda.synchronize()
        assert torch.equal(o_d, o_s) and torch.equal(lse_d, lse_s), (B, N)


def test_two_streams(device, lib):
    """Concurrent calls on two streams, each with its own workspace."""
    q, k, v = seeded((2, 32, 1300, 128), 20, device), seeded((2, 8, 1300, 128), 21, device), \
        seeded((2, 8, 1300, 128), 22, device)
    q2, k2, v2 = seeded((1, 64, 1200, 64), 23, device), seeded((1, 8, 1200, 64), 24, device), \
        seeded((1, 8, 1200, 64), 25, device)
    o_s, _ = run(lib, q, k, v, 1)
    o2_s, _ = run(lib, q2, k2, v2, 0)
    torch.cuda.synchronize()
    s1, s2 = torch.cuda.Stream(device), torch.cuda.Stream(device)
    ws1 = workspace_for(lib, q, k, 1, device)
    ws2 = workspace_for(lib, q2, k2, 0, device)
    torch.cuda.synchronize()
    outs = []
    for _ in range(3):
        outs.append((run(lib, q, k, v, 1, workspace=ws1, stream=s1)[0],
                     run(lib, q2, k2, v2, 0, workspace=ws2, stream=s2)[0]))
    torch.cuda.synchronize()
    for o1, o2 in outs:
        assert torch.equal(o1, o_s) and torch.equal(o2, o2_s)


def test_binding_uses_dynamic_path(device, lib):
    """The binding hands the counter workspace over: under policy DYNAMIC,
    calls through flash_attention_forward agree bitwise with the static run;
    so do AUTO calls long enough for its long-launch rule (C5's shape)."""
    q, k, v = seeded((1, 32, 4096, 128), 30, device), seeded((1, 8, 4096, 128), 31, device), \
        seeded((1, 8, 4096, 128), 32, device)
    o_s, _ = run(lib, q, k, v, 1)
    _C.set_kernel_policy(3)
    try:
        o_b = _C.flash_attention_forward(q, k, v, True, 1.0 / math.sqrt(128))
    finally:
        _C.set_kernel_policy(0)
    torch.cuda.synchronize()
    assert torch.equal(o_b, o_s)
    q, k, v = seeded((2, 64, 16384, 128), 33, device), seeded((2, 8, 16384, 128), 34, device), \
        seeded((2, 8, 16384, 128), 35, device)
    o_s, _ = run(lib, q, k, v, 1)
    lib.fa_sm75_set_kernel_policy(0)
    o_b = _C.flash_attention_forward(q, k, v, True, 1.0 / math.sqrt(128))
    torch.cuda.synchronize()
    assert torch.equal(o_b, o_s)
