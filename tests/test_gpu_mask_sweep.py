"""Seeded sweep of structured boolean masks through the kernels (forward O and
LSE; gradients for Nq <= 400 and Nk <= 800), against the numpy oracle at the
bars of tests/sweep_checks.py.

Each case draws, from a fixed seed, a batch, KV heads and GQA group, query and
key lengths, head_dim 64 or 128, binary16 or bfloat16, a causal mode applied
together with the mask (none, top-left, bottom-right: key j reaches query i
iff both allow it), and one mask structure of those that reach the kernels
from transformers and serving code:
  * causal_pad: the causal mask of a padded prefill as transformers
    materialises it, [B, 1, Nq, Nk], bottom-right aligned, with left or right
    padding of a different length per sequence (left padding leaves the
    padded query rows with no visible key);
  * band: a sliding window per row (bottom-right aligned), [Nq, Nk] or
    [1, 1, Nq, Nk] shared, or [B, 1, Nq, Nk] with a window per sequence;
  * holes: causal or full rows with 10% of their keys hidden at random and
    about 5% of the rows empty, [B, 1, Nq, Nk];
  * key_pad: a key-padding mask [B, 1, 1, Nk] (a visible prefix per
    sequence, sometimes empty), which the kernels read in place as bytes;
  * per_head_band: a window per query head, [B, Hq, Nq, Nk].
These are the mask kinds the packing kernel's row spans and dense-row flags
are built for (tiles outside every row's span skipped, tiles inside every
row's interval read without mask words), so the sweep crosses those paths
with the sequence ends, the causal diagonal and grouped heads.

FA_MASK_SWEEP_CASES draws more cases (the default run keeps 40).
"""
import os

import numpy as np
import pytest
import torch

from sweep_checks import check_case

pytestmark = pytest.mark.gpu

N_CASES = int(os.environ.get("FA_MASK_SWEEP_CASES", "40"))
KINDS = ("causal_pad", "band", "holes", "key_pad", "per_head_band")


def draw(case):
    rng = np.random.default_rng(7000 + case)
    B = int(rng.integers(1, 4))
    Hkv = int(rng.choice([1, 2, 4]))
    Hq = Hkv * int(rng.choice([1, 2, 4, 7]))
    Nq = int(rng.choice([1, 2, 3])) if rng.random() < 0.2 else int(rng.integers(1, 700))
    Nk = Nq if rng.random() < 0.5 else int(rng.integers(max(1, Nq // 2), 2500))
    D = int(rng.choice([64, 128]))
    bf16 = bool(rng.random() < 0.3)
    code = int(rng.choice([0, 0, 1, 2]))
    kind = KINDS[int(rng.integers(0, len(KINDS)))]
    return rng, B, Hq, Hkv, Nq, Nk, D, bf16, code, kind


def build_mask(rng, kind, B, Hq, Nq, Nk):
    """The case's mask as a numpy bool array (True = visible)."""
    i = np.arange(Nq)[:, None]
    j = np.arange(Nk)[None, :]
    off = Nk - Nq  # bottom-right alignment, as transformers lays out a prefill over a cache
    causal = j <= i + off
    if kind == "causal_pad":
        left = bool(rng.random() < 0.5)
        m = np.empty((B, 1, Nq, Nk), dtype=bool)
        for b in range(B):
            p = int(rng.integers(0, Nk // 2 + 1))
            keys = (j >= p) if left else (j < Nk - p)
            m[b, 0] = causal & keys
        return m
    if kind == "band":
        layout = int(rng.integers(0, 3))
        if layout < 2:
            w = int(rng.integers(1, Nk + 1))
            m = causal & (j > i + off - w)
            return m if layout == 0 else m[None, None]
        m = np.empty((B, 1, Nq, Nk), dtype=bool)
        for b in range(B):
            w = int(rng.integers(1, Nk + 1))
            m[b, 0] = causal & (j > i + off - w)
        return m
    if kind == "holes":
        base = causal if rng.random() < 0.5 else np.ones((Nq, Nk), dtype=bool)
        m = base[None, None] & (rng.random((B, 1, Nq, Nk)) > 0.1)
        m &= ~(rng.random((B, 1, Nq, 1)) < 0.05)
        return m
    if kind == "key_pad":
        m = np.zeros((B, 1, 1, Nk), dtype=bool)
        for b in range(B):
            n = 0 if rng.random() < 0.05 else int(rng.integers(1, Nk + 1))
            m[b, 0, 0, :n] = True
        return m
    m = np.empty((B, Hq, Nq, Nk), dtype=bool)  # per_head_band
    for b in range(B):
        for h in range(Hq):
            w = int(rng.integers(1, Nk + 1))
            m[b, h] = causal & (j > i + off - w)
    return m


@pytest.mark.parametrize("case", range(N_CASES))
def test_mask_case(device, case):
    rng, B, Hq, Hkv, Nq, Nk, D, bf16, code, kind = draw(case)
    mask = torch.from_numpy(build_mask(rng, kind, B, Hq, Nq, Nk))
    dt = torch.bfloat16 if bf16 else torch.float16
    g = torch.Generator("cpu").manual_seed(7000 + case)
    q = torch.randn(B, Hq, Nq, D, generator=g).to(dt)
    k = torch.randn(B, Hkv, Nk, D, generator=g).to(dt)
    v = torch.randn(B, Hkv, Nk, D, generator=g).to(dt)
    print(f"[mask sweep {case}] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={code} "
          f"{'bf16' if bf16 else 'fp16'} kind={kind} mask={tuple(mask.shape)} "
          f"visible={float(mask.float().mean()):.3f}", flush=True)
    check_case(device, q, k, v, mask, code, None, bf16, g)
