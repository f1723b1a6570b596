"""fa_sm75_forward_noalloc: the forward with the library's own static scratch
instead of a caller workspace (needs a GPU).

Checked through the C ABI against fa_sm75_forward given a workspace of
fa_sm75_workspace_size() bytes: bitwise equal outputs and LSE, on two calls
in a row where the second is smaller (the scratch keeps the first call's
contents), for the two paths that use scratch: the split-K decode kernel
(partials; also with a key-padding mask read as bytes) and the fused
kernel's dynamic schedule (queue counters); and a HIP graph whose capture
holds the process's first noalloc call, replayed against eager calls.
"""
import ctypes

import pytest
import torch

from capi_types import LIB, Params

pytestmark = pytest.mark.gpu

FA_OK, FA_ERR_INVALID_ARGUMENT = 0, 1
FA_POLICY_AUTO, FA_POLICY_DYNAMIC = 0, 3


@pytest.fixture(scope="module")
def lib():
    lib = ctypes.CDLL(LIB)
    for n in ("fa_sm75_forward", "fa_sm75_forward_noalloc"):
        getattr(lib, n).argtypes = [ctypes.POINTER(Params)]
        getattr(lib, n).restype = ctypes.c_int
    lib.fa_sm75_workspace_size.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.restype = ctypes.c_int64
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    lib.fa_sm75_set_kernel_policy.restype = ctypes.c_int
    return lib


def call_pair(lib, device, B, Hq, Hkv, Nq, Nk, D, causal, seed, key_mask=False):
    """Runs one problem through both entry points; returns the two (O, LSE)
    pairs and the workspace size the call asks for.  key_mask: a random
    [B, Nk] key-padding mask given as bytes (mask_keys)."""
    print(f"[noalloc] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal} "
          f"key_mask={key_mask}", flush=True)
    g = torch.Generator("cpu").manual_seed(seed)
    q = torch.randn(B, Hq, Nq, D, generator=g).half().to(device)
    k = torch.randn(B, Hkv, Nk, D, generator=g).half().to(device)
    v = torch.randn(B, Hkv, Nk, D, generator=g).half().to(device)
    keys = (torch.rand(B, Nk, generator=g) < 0.8).to(device) if key_mask else None
    outs = []
    need = None
    for entry in ("fa_sm75_forward", "fa_sm75_forward_noalloc"):
        o = torch.full_like(q, float("nan"))
        lse = torch.full((B, Hq, Nq), float("nan"), dtype=torch.float32, device=device)
        p = Params()
        p.q, p.k, p.v, p.o, p.lse = (q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr(),
                                     lse.data_ptr())
        p.batch, p.heads_q, p.heads_kv, p.seq_len, p.seq_len_kv, p.head_dim = (
            B, Hq, Hkv, Nq, Nk, D)
        lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
        p.scale, p.causal = D ** -0.5, causal
        p.stream = torch.cuda.current_stream().cuda_stream
        if keys is not None:
            p.mask_keys, p.mask_keys_stride_b, p.mask_keys_stride_k = keys.data_ptr(), Nk, 1
        ws = None
        if entry == "fa_sm75_forward":
            need = lib.fa_sm75_workspace_size(ctypes.byref(p))
            ws = torch.empty(max(need, 16), dtype=torch.uint8, device=device)
            p.workspace, p.workspace_bytes = ws.data_ptr(), need
        rc = getattr(lib, entry)(ctypes.byref(p))
        assert rc == FA_OK, (entry, lib.fa_sm75_last_error())
        torch.cuda.synchronize()
        del ws
        outs.append((o, lse))
    return outs, need


def assert_same(outs):
    (o1, l1), (o2, l2) = outs
    assert torch.equal(o1, o2)
    assert torch.equal(l1, l2)
    assert not torch.isnan(o2).any()


def test_first_call_under_graph_capture(device, lib):
    """The first fa_sm75_forward_noalloc call of the process is made while a
    HIP graph is being captured (it runs first in this module, and no other
    test makes a noalloc call that reaches the scratch): the per-device
    scratch lookup happens inside the capture.  The graph (split-K decode
    shape: partials in the scratch) is replayed three times on inputs
    rewritten in place, with eager work between the replays, and each replay
    is bitwise the eager fa_sm75_forward with a workspace on the same
    inputs."""
    B, Hq, Hkv, Nq, Nk, D = 2, 32, 8, 1, 4096, 128
    print(f"[noalloc graph] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D}", flush=True)
    q = torch.empty(B, Hq, Nq, D, dtype=torch.float16, device=device)
    k = torch.empty(B, Hkv, Nk, D, dtype=torch.float16, device=device)
    v = torch.empty_like(k)
    o_graph = torch.full_like(q, float("nan"))
    o_eager = torch.full_like(q, float("nan"))

    def params(o, stream):
        p = Params()
        p.q, p.k, p.v, p.o = q.data_ptr(), k.data_ptr(), v.data_ptr(), o.data_ptr()
        p.batch, p.heads_q, p.heads_kv, p.seq_len, p.seq_len_kv, p.head_dim = (
            B, Hq, Hkv, Nq, Nk, D)
        lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
        p.scale, p.stream = D ** -0.5, stream
        return p

    def fill(seed):
        g = torch.Generator("cpu").manual_seed(seed)
        for t in (q, k, v):
            t.copy_(torch.randn(t.shape, generator=g).half())

    def eager():
        p = params(o_eager, torch.cuda.current_stream().cuda_stream)
        need = lib.fa_sm75_workspace_size(ctypes.byref(p))
        assert need > 0  # the split-K partials
        ws = torch.empty(need, dtype=torch.uint8, device=device)
        p.workspace, p.workspace_bytes = ws.data_ptr(), need
        assert lib.fa_sm75_forward(ctypes.byref(p)) == FA_OK, lib.fa_sm75_last_error()
        torch.cuda.synchronize()
        return o_eager.clone()

    fill(1)
    eager()  # the library's kernels are loaded before the capture
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = lib.fa_sm75_forward_noalloc(
            ctypes.byref(params(o_graph, torch.cuda.current_stream().cuda_stream)))
    assert rc == FA_OK, lib.fa_sm75_last_error()
    for rep in range(3):
        fill(10 + rep)
        graph.replay()
        junk = torch.randn(1 << 20, device=device).sum()  # eager work between replays
        torch.cuda.synchronize()
        want = eager()
        assert torch.isfinite(junk)
        assert not torch.isnan(o_graph).any()
        assert torch.equal(o_graph, want), rep


def test_split_k_partials_in_scratch(device, lib):
    # group * Nq <= 32: split-K decode; the partials go to the scratch
    outs, need = call_pair(lib, device, 2, 32, 8, 1, 4096, 128, 0, seed=1)
    assert need > 0
    assert_same(outs)
    outs, need2 = call_pair(lib, device, 1, 8, 2, 3, 700, 64, 2, seed=2)  # smaller
    assert 0 < need2 < need
    assert_same(outs)


def test_split_k_with_key_padding_mask(device, lib):
    # the same, with a key-padding mask read as bytes
    outs, need = call_pair(lib, device, 4, 14, 2, 1, 6000, 64, 0, seed=5, key_mask=True)
    assert need > 0
    assert_same(outs)
    outs, need2 = call_pair(lib, device, 2, 8, 2, 1, 1500, 128, 2, seed=6, key_mask=True)
    assert 0 < need2 < need
    assert_same(outs)


def test_dynamic_schedule_counters_in_scratch(device, lib):
    assert lib.fa_sm75_set_kernel_policy(FA_POLICY_DYNAMIC) == FA_OK
    try:
        outs, need = call_pair(lib, device, 1, 16, 4, 2048, 2048, 128, 1, seed=3)
        assert need > 0
        assert_same(outs)
        outs, _ = call_pair(lib, device, 1, 8, 8, 700, 700, 64, 1, seed=4)  # smaller
        assert_same(outs)
    finally:
        lib.fa_sm75_set_kernel_policy(FA_POLICY_AUTO)


def test_rejects_a_workspace(device, lib):
    q = torch.zeros(1, 2, 64, 64, dtype=torch.float16, device=device)
    p = Params()
    p.q = p.k = p.v = p.o = q.data_ptr()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = 1, 2, 2, 64, 64
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.scale = 0.125
    p.workspace, p.workspace_bytes = q.data_ptr(), 1024
    assert lib.fa_sm75_forward_noalloc(ctypes.byref(p)) == FA_ERR_INVALID_ARGUMENT
    assert b"takes no workspace" in lib.fa_sm75_last_error()
