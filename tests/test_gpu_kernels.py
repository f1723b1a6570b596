"""The fused kernel shapes against the oracle on the same inputs (needs a GPU).

The prefill kernel comes as 128-row workgroups of 4 waves (two per CU, K/V
double-buffered; the automatic choice for most launches), 256-row workgroups
of 8 waves (one per CU, K/V triple-buffered at head_dim 64, double-buffered
at 128) and 128-row workgroups of 8
waves whose two groups of 4 split the block's key tiles and merge through LDS
(one per CU; the automatic choice for launches whose blocks all get a CU at
once), and the paired form of the latter for causal head_dim-64 launches
(blocks i and nqb-1-i of one head on one workgroup, their key tiles dealt
evenly to the two groups; the automatic choice where the pairs all get a CU
at once);
fa_sm75_set_kernel_policy forces each, so each is checked on the same shapes,
including the tails, odd tile counts and 1-row cases the split-K path would
otherwise take.  Tolerance as in test_gpu_parity:
|O - O_ref| <= 2e-3 + 1e-2 |O_ref|.
"""
import contextlib
import ctypes

import numpy as np
import pytest
import torch

from capi_types import LIB
from flash_attention_sm75 import flash_attention_forward, flash_attention_forward_lse
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

NARROW, WIDE, SPLIT, PAIRS = 1, 2, 4, 5


@contextlib.contextmanager
def policy(p):
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    assert lib.fa_sm75_set_kernel_policy(p) == 0
    try:
        yield
    finally:
        lib.fa_sm75_set_kernel_policy(0)


def inputs(B, Hq, Hkv, N, D, seed, std=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    q = (torch.randn(B, Hq, N, D, generator=g) * std).half()
    k = (torch.randn(B, Hkv, N, D, generator=g) * std).half()
    v = (torch.randn(B, Hkv, N, D, generator=g) * std).half()
    return q, k, v


def check(out, q, k, v, causal, scale=None, label=""):
    expect = ref.attention_reference_chunked(q.numpy(), k.numpy(), v.numpy(), causal=causal,
                                             scale=scale, return_f32=True)
    res = ref.check_correctness(out.float().cpu().numpy(), expect, atol=2e-3, rtol=1e-2)
    print(f"  {label}: max_abs={res['max_abs_err']:.3e}", flush=True)
    assert res["allclose"], res


SHAPES = [
    # B, Hq, Hkv, N, D, causal
    (1, 2, 2, 1, 128, False),
    (1, 2, 2, 63, 128, True),
    (1, 2, 1, 200, 128, True),
    (1, 4, 2, 256, 128, False),
    (1, 4, 1, 257, 128, True),
    (2, 8, 2, 511, 128, True),
    (1, 4, 4, 700, 128, False),
    (1, 3, 1, 1030, 128, True),
    (1, 2, 2, 300, 64, True),
    (2, 4, 2, 777, 64, False),
    (1, 8, 8, 1100, 64, True),
    (3, 5, 1, 129, 64, False),
    (1, 2, 2, 65, 64, True),
    (1, 2, 2, 130, 128, False),      # 3 key tiles: odd split
    (4, 8, 8, 2048, 64, True),       # C3
    # single-round causal launches, whose blocks are laid out in pairs
    (1, 36, 3, 1700, 64, True),      # one sequence (3 units), 504 blocks
    (2, 16, 8, 2000, 128, True),     # 8 sequences, exactly 512 blocks
    (1, 24, 8, 2048, 64, True),      # 8 sequences, 384 blocks (half the pairs)
]


@pytest.mark.parametrize("pol", [NARROW, WIDE, SPLIT, PAIRS],
                         ids=["narrow", "wide", "split", "pairs"])
@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal", SHAPES)
def test_forced_policy(device, pol, B, Hq, Hkv, N, D, causal):
    print(f"[policy {pol}] B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal}", flush=True)
    q, k, v = inputs(B, Hq, Hkv, N, D, seed=N + 7 * Hq)
    with policy(pol):
        out = flash_attention_forward(q.to(device), k.to(device), v.to(device), causal=causal)
        torch.cuda.synchronize()
    check(out, q, k, v, causal, label=f"pol{pol} N{N} D{D}")


@pytest.mark.parametrize("pol", [NARROW, WIDE, SPLIT, PAIRS],
                         ids=["narrow", "wide", "split", "pairs"])
@pytest.mark.parametrize("scale", [0.0, -0.1, 1.0])
@pytest.mark.parametrize("D", [64, 128])
def test_forced_policy_scales_and_lse(device, pol, scale, D):
    q, k, v = inputs(1, 4, 2, 333, D, seed=5)
    with policy(pol):
        out, lse = flash_attention_forward_lse(q.to(device), k.to(device), v.to(device),
                                               causal=True, scale=scale)
        torch.cuda.synchronize()
    check(out, q, k, v, True, scale=scale, label=f"pol{pol} scale{scale}")
    lse_ref = ref.attention_lse(q.numpy(), k.numpy(), causal=True, scale=scale)
    np.testing.assert_allclose(lse.cpu().numpy(), lse_ref, atol=2e-4, rtol=1e-5)


def test_key_split_auto_picks_one(device):
    """The automatic choice equals a forced kernel bit for bit: key-split
    workgroups on launches whose blocks all get a CU and on small causal
    launches at head_dim 128, paired key-split workgroups on causal
    head_dim-64 launches whose pairs of blocks all get a CU (rows of at
    least 32 blocks), 128-row ones otherwise; the kernels differ only by the
    merge's rounding."""
    for (B, Hq, Hkv, N, D) in ((1, 4, 4, 4200, 128), (4, 8, 8, 2048, 64), (2, 32, 8, 2048, 128),
                               (1, 8, 8, 4096, 64), (1, 16, 16, 4096, 64), (2, 48, 8, 1024, 64)):
        q, k, v = (t.to(device) for t in inputs(B, Hq, Hkv, N, D, seed=B + N + D))
        outs = {}
        for pol in (0, NARROW, SPLIT, PAIRS):
            with policy(pol):
                outs[pol] = flash_attention_forward(q, k, v, causal=True)
        torch.cuda.synchronize()
        assert any(torch.equal(outs[0], outs[p]) for p in (NARROW, SPLIT, PAIRS))
        for p in (SPLIT, PAIRS):
            diff = (outs[NARROW].float() - outs[p].float()).abs().max().item()
            assert diff < 4e-3, (p, diff)


# The paired key split at its edges: one block (no pair), a pair whose
# larger block fills group 0 so group 1 starts in the smaller one, a middle
# block of an odd count, ragged lengths, bottom-right alignment with the
# query block rows past the keys and with blocks that see no key, GQA, and
# bfloat16; O and LSE against the oracle.
PAIR_CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal, bf16
    (1, 4, 2, 1, 1, 64, True, False),
    (1, 2, 2, 129, 129, 64, True, False),
    (1, 2, 2, 384, 384, 64, True, False),
    (2, 3, 1, 1000, 1000, 64, True, False),
    (1, 4, 2, 300, 1000, 64, "bottom_right", False),
    (1, 4, 4, 1000, 300, 64, "bottom_right", False),
    (1, 2, 2, 700, 900, 64, True, False),
    (2, 8, 2, 1500, 1500, 64, True, True),
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal,bf16", PAIR_CASES)
def test_split_pairs_edges(device, B, Hq, Hkv, Nq, Nk, D, causal, bf16):
    from flash_attention_sm75 import flash_attention_forward_ex
    print(f"[pairs] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal} bf16={bf16}",
          flush=True)
    dt = torch.bfloat16 if bf16 else torch.float16
    g = torch.Generator("cpu").manual_seed(Nq + 3 * Nk)
    q, k, v = (torch.randn(B, h, n, D, generator=g).to(dt)
               for h, n in ((Hq, Nq), (Hkv, Nk), (Hkv, Nk)))
    with policy(PAIRS):
        o, lse = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                            causal=causal, return_lse=True)
        torch.cuda.synchronize()
    code = {True: 1, "bottom_right": 2}[causal]
    npf = lambda t: t.float().numpy()
    want = ref.attention_reference(npf(q), npf(k), npf(v), causal=code, return_f32=True)
    got = o.float().cpu().numpy()
    if bf16:
        spv = ref.attention_f64(npf(q), npf(k), np.abs(npf(v)), causal=code)
        bound = 2.0 ** -8 * (spv + 2 * np.abs(want)) * 1.01 + 2e-6
    else:
        bound = 2e-3 + 1e-2 * np.abs(want)
    err = np.abs(got - want)
    print(f"  O max_abs={err.max():.3e} worst/bound={(err / bound).max():.3f}", flush=True)
    assert np.all(err <= bound)
    lse_ref = ref.attention_lse(npf(q), npf(k), causal=code)
    got_lse = lse.cpu().numpy()
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(got_lse), fin)
    tol = 2e-4 if not bf16 else float(np.log1p(2.0 ** -8)) + 1e-5
    np.testing.assert_allclose(got_lse[fin], lse_ref[fin], atol=tol, rtol=1e-5)


def test_kernels_agree_and_auto_picks_one(device):
    """On a large causal launch auto mode equals one of the forced kernels bit
    for bit; a small one (12 query blocks) runs the split-K small-launch path
    (oracle-checked in test_gpu_small_launch.py) and agrees with them within
    rounding; the forced kernels agree within rounding."""
    for (B, Hq, Hkv, N) in ((4, 32, 8, 1000), (1, 4, 4, 300)):
        q, k, v = (t.to(device) for t in inputs(B, Hq, Hkv, N, 128, seed=B * N))
        outs = {}
        for pol in (0, NARROW, WIDE, SPLIT):
            with policy(pol):
                outs[pol] = flash_attention_forward(q, k, v, causal=True)
        torch.cuda.synchronize()
        small = B * Hq * ((N + 127) // 128) <= 64
        if small:
            diff = (outs[0].float() - outs[NARROW].float()).abs().max().item()
            assert diff < 4e-3, diff
        else:
            assert any(torch.equal(outs[0], outs[p]) for p in (NARROW, WIDE, SPLIT))
        for p in (WIDE, SPLIT):
            diff = (outs[NARROW].float() - outs[p].float()).abs().max().item()
            assert diff < 4e-3, (p, diff)
