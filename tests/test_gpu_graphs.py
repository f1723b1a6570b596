"""The forward paths captured in HIP graphs (torch.cuda.CUDAGraph) and replayed.

Serving loops capture attention into graphs.  Every path records only kernel
launches on the capturing stream (the dynamic schedule clears its counters
with a kernel, not a memset; workspaces come from torch's allocator, which
serves captures from the graph's private pool).  Each case captures one
call, then replays it three times with fresh data copied into the captured
inputs and unrelated eager work in between, and checks every replay bitwise
against an eager call on the same data.  Masked calls are captured with the
mask too (key-padding bytes read in place, or a per-row mask packed by a
kernel inside the graph) and the mask is rewritten between replays.
"""
import ctypes

import pytest
import torch

from capi_types import LIB
from flash_attention_sm75 import flash_attention_forward, flash_attention_forward_ex

pytestmark = pytest.mark.gpu


def set_policy(p):
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    assert lib.fa_sm75_set_kernel_policy(p) == 0


def fill(tensors, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    for t in tensors:
        t.copy_(torch.randn(t.shape, generator=g).half())


CASES = [
    # id, policy, (B, Hq, Hkv, Nq, Nk, D), causal
    ("static", 1, (1, 8, 2, 1000, 1000, 128), True),
    ("dynamic", 3, (2, 32, 8, 1100, 1100, 64), True),
    ("key-split", 4, (1, 8, 8, 2100, 2100, 128), True),
    ("auto", 0, (1, 4, 4, 300, 300, 64), False),
    ("decode split-K", 0, (4, 32, 8, 1, 4096, 128), False),
]


@pytest.mark.parametrize("name,pol,shape,causal", CASES, ids=[c[0] for c in CASES])
def test_graph_replays_match_eager(device, name, pol, shape, causal):
    B, Hq, Hkv, Nq, Nk, D = shape
    q = torch.empty(B, Hq, Nq, D, dtype=torch.float16, device=device)
    k = torch.empty(B, Hkv, Nk, D, dtype=torch.float16, device=device)
    v = torch.empty_like(k)
    fill((q, k, v), 1)

    def call():
        if Nq == Nk:
            return flash_attention_forward(q, k, v, causal=causal)
        return flash_attention_forward_ex(q, k, v, causal=causal)

    set_policy(pol)
    try:
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(2):
                call()  # warm-up outside the capture
        torch.cuda.current_stream().wait_stream(side)
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            out = call()
        for rep in range(3):
            fill((q, k, v), 10 + rep)
            graph.replay()
            junk = torch.randn(1 << 20, device=device).sum()  # eager work between replays
            torch.cuda.synchronize()
            expect = call()
            torch.cuda.synchronize()
            assert torch.isfinite(junk)
            assert torch.equal(out, expect), (name, rep)
    finally:
        set_policy(0)


MASK_CASES = [
    # id, (B, Hq, Hkv, Nq, Nk, D), mask shape, causal
    ("key padding, decode", (4, 14, 2, 1, 3000, 64), (4, 1, 1, 3000), False),
    ("key padding, prefill", (2, 8, 2, 700, 700, 128), (2, 1, 1, 700), True),
    ("per-row mask, decode", (2, 8, 2, 4, 2000, 128), (2, 8, 4, 2000), "bottom_right"),
]


@pytest.mark.parametrize("name,shape,mshape,causal", MASK_CASES, ids=[c[0] for c in MASK_CASES])
def test_graph_replays_with_mask(device, name, shape, mshape, causal):
    """A boolean mask captured with the call: a key-padding mask's bytes are
    read in place at every replay, a per-row mask is packed by a kernel that
    is part of the graph; either way a mask rewritten in place between
    replays takes effect, bitwise as in an eager call."""
    B, Hq, Hkv, Nq, Nk, D = shape
    q = torch.empty(B, Hq, Nq, D, dtype=torch.float16, device=device)
    k = torch.empty(B, Hkv, Nk, D, dtype=torch.float16, device=device)
    v = torch.empty_like(k)
    mask = torch.empty(mshape, dtype=torch.bool, device=device)
    fill((q, k, v), 1)

    def fill_mask(seed):
        g = torch.Generator("cpu").manual_seed(seed)
        m = torch.rand(mshape, generator=g) < 0.7
        m[..., 0] = True
        mask.copy_(m)

    fill_mask(2)

    def call():
        return flash_attention_forward_ex(q, k, v, causal=causal, attn_mask=mask)

    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    previous = None
    for rep in range(3):
        fill((q, k, v), 10 + rep)
        fill_mask(20 + rep)
        graph.replay()
        junk = torch.randn(1 << 20, device=device).sum()
        torch.cuda.synchronize()
        expect = call()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        assert torch.equal(out, expect), (name, rep)
        if previous is not None:
            assert not torch.equal(out, previous)
        previous = out.clone()
