"""The backward kernels (dQ, dK, dV) against the float64 oracle (needs a GPU).

No reference counterpart: the reference's backward raises
(src/flash_attention_sm75/ops.py:47-52).  The oracle
(attention_backward_f64, pinned in test_oracle_backward.py) is the exact
gradient of the same fp16/bf16 inputs.  The kernels round P and dS to the
element type before the products that take them (as the forward rounds P;
the dK/dV kernel forms dS from that rounded P), use the rounded forward
output in rowsum(dO o O), and round the gradients;
each of those is a relative 2^-11 (binary16) or 2^-8 (bfloat16) error on
terms of mixed sign.  Bar, per gradient tensor G against its oracle R:
    |G - R| <= ATOL * max|R| + RTOL * |R|   elementwise,
binary16 ATOL = 2e-3, RTOL = 1e-2 (the forward's bar, with the absolute
term relative to the gradient's scale); bfloat16 ATOL = 1e-2, RTOL = 4e-2
(the 8x coarser rounding).  Observed: up to 0.2 (binary16) and 0.35
(bfloat16) of the bar; max|R| is floored at 1e-2, since a gradient
that is exactly zero (dQ with a single key) comes out as rounding noise of
the P(dP - rowsum) cancellation.  At sizes the oracle cannot reach, two exact
identities of the gradient are checked instead: the keys' dK rows sum to
zero, and the keys' dV rows sum to the dO rows of the group's queries.
"""
import numpy as np
import pytest
import torch

import flash_attn_sm75_cuda as _C
from flash_attention_sm75 import (flash_attention, flash_attention_backward,
                                  flash_attention_forward, flash_attention_forward_ex)
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

BAR = {torch.float16: (2e-3, 1e-2), torch.bfloat16: (1e-2, 4e-2)}
CODE = {False: 0, True: 1, "bottom_right": 2}


def seeded(shape, seed, dtype=torch.float16):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g).to(dtype)


def npf(t):
    return t.float().cpu().numpy()


def run_backward(q, k, v, do, causal, device, scale=None):
    qd, kd, vd, dod = (t.to(device) for t in (q, k, v, do))
    o, lse = flash_attention_forward_ex(qd, kd, vd, causal=causal, scale=scale, return_lse=True)
    grads = flash_attention_backward(dod, qd, kd, vd, o, lse, causal=causal, scale=scale)
    torch.cuda.synchronize()
    return grads


def assert_grads(grads, want, dtype, label):
    atol, rtol = BAR[dtype]
    for name, g, w in zip(("dQ", "dK", "dV"), grads, want):
        g = npf(g)
        scale = max(float(np.abs(w).max()) if w.size else 0.0, 1e-2)
        err = np.abs(g - w)
        worst = float((err / (atol * scale + rtol * np.abs(w) + 1e-30)).max()) if w.size else 0.0
        print(f"  {label} {name}: max_abs={err.max() if err.size else 0:.3e} "
              f"max|R|={scale:.3e} worst/bar={worst:.3f}", flush=True)
        assert np.isfinite(g).all(), name
        assert worst <= 1.0, (name, worst)


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal
    (1, 2, 2, 128, 128, 64, False),
    (1, 2, 2, 128, 128, 128, True),
    (1, 4, 2, 200, 200, 128, True),      # ragged tail, GQA 2:1
    (2, 8, 2, 333, 333, 64, True),       # GQA 4:1, odd length
    (2, 3, 3, 1, 1, 128, False),         # single row
    (1, 4, 1, 513, 513, 64, False),      # MQA, one row past a block
    (1, 4, 4, 100, 260, 128, "bottom_right"),
    (1, 2, 1, 300, 77, 64, "bottom_right"),  # rows that see no key
    (1, 2, 2, 70, 300, 128, True),       # top-left with Nq < Nk: keys no query sees
    (1, 8, 8, 1024, 1024, 128, True),
    # dQ kernel: key tiles no row of a query block masks (below its diagonal,
    # inside the keys) run in a loop of their own; with these diagonals that
    # loop ends after an even or an odd number of tiles, depending on the block
    (1, 2, 1, 200, 600, 64, "bottom_right"),
    (1, 4, 2, 150, 500, 128, "bottom_right"),
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", CASES)
def test_backward_matches_oracle(device, B, Hq, Hkv, Nq, Nk, D, causal):
    print(f"[bwd] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal}", flush=True)
    q, k, v = seeded((B, Hq, Nq, D), 1), seeded((B, Hkv, Nk, D), 2), seeded((B, Hkv, Nk, D), 3)
    do = seeded((B, Hq, Nq, D), 4)
    grads = run_backward(q, k, v, do, causal, device)
    want = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), causal=CODE[causal])
    assert_grads(grads, want, torch.float16, f"Nq{Nq} Nk{Nk} D{D}")


# The dK/dV kernel runs its two roles in periods (one per step = one 64-row
# query tile of one query head), unrolled by three with one or two periods
# left over: these shapes give every step count from 1 to 8 and 12 for one
# 128-key block (steps = heads per KV head x query tiles).
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("Hq,Hkv,Nq", [(1, 1, 64), (1, 1, 128), (1, 1, 192), (1, 1, 256),
                                       (1, 1, 300), (3, 1, 128), (7, 7, 448), (2, 1, 256),
                                       (4, 1, 192)])
def test_backward_period_counts(device, Hq, Hkv, Nq, D):
    print(f"[bwd periods] Hq={Hq} Hkv={Hkv} Nq={Nq} Nk=128 D={D}", flush=True)
    q, k, v = seeded((1, Hq, Nq, D), 11), seeded((1, Hkv, 128, D), 12), seeded((1, Hkv, 128, D), 13)
    do = seeded((1, Hq, Nq, D), 14)
    grads = run_backward(q, k, v, do, False, device)
    want = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), causal=0)
    assert_grads(grads, want, torch.float16, f"Hq{Hq} Nq{Nq} D{D}")


# Rows that see one or two keys of a peaked softmax (scale 0.3): dP - rowsum
# nearly cancels there, so the rounding of the forward's O, which the row
# term rowsum(dO o O) takes, moves dQ and dK by up to about 1.5e-3 of their
# scale against the exact gradient (beyond the bar; a randomized sweep found
# such a case).  The bar holds against the same closed form with the row term
# taken from the kernel's own O (attention_backward_f64's delta_from_o), which
# leaves the kernels' own arithmetic: measured 1.2-1.5e-4 there.
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", [
    (1, 4, 4, 2, 215, 64, True),             # top-left: the rows see 1 and 2 keys
    (2, 8, 2, 40, 12, 128, "bottom_right"),  # Nq > Nk: rows see 0 to 12 keys
    (1, 6, 3, 3, 3, 64, True),
])
def test_backward_few_keys_peaked(device, dtype, B, Hq, Hkv, Nq, Nk, D, causal):
    print(f"[bwd peaked] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal} {dtype}",
          flush=True)
    q, k, v = (seeded(s, i, dtype) for i, s in enumerate(((B, Hq, Nq, D), (B, Hkv, Nk, D),
                                                          (B, Hkv, Nk, D)), 31))
    do = seeded((B, Hq, Nq, D), 34, dtype)
    qd, kd, vd, dod = (t.to(device) for t in (q, k, v, do))
    o, lse = flash_attention_forward_ex(qd, kd, vd, causal=causal, scale=0.3, return_lse=True)
    grads = flash_attention_backward(dod, qd, kd, vd, o, lse, causal=causal, scale=0.3)
    torch.cuda.synchronize()
    args = (npf(q), npf(k), npf(v), npf(do))
    want = ref.attention_backward_f64(*args, causal=CODE[causal], scale=0.3, delta_from_o=npf(o))
    assert_grads(grads, want, dtype, f"Nq{Nq} Nk{Nk} D{D} (row term from O)")
    exact = ref.attention_backward_f64(*args, causal=CODE[causal], scale=0.3)
    for name, g, w in zip(("dQ", "dK", "dV"), grads, exact):
        print(f"  against the exact gradient {name}: max_abs={np.abs(npf(g) - w).max():.3e} "
              f"max|R|={np.abs(w).max():.3e}", flush=True)


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", [
    (1, 4, 2, 200, 200, 128, True),
    (2, 4, 1, 150, 150, 64, False),
    (1, 2, 2, 90, 170, 64, "bottom_right"),
])
def test_backward_bf16(device, B, Hq, Hkv, Nq, Nk, D, causal):
    print(f"[bwd bf16] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal}", flush=True)
    bf = torch.bfloat16
    q, k, v = seeded((B, Hq, Nq, D), 5, bf), seeded((B, Hkv, Nk, D), 6, bf), seeded((B, Hkv, Nk, D), 7, bf)
    do = seeded((B, Hq, Nq, D), 8, bf)
    grads = run_backward(q, k, v, do, causal, device)
    assert all(g.dtype == bf for g in grads)
    want = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), causal=CODE[causal])
    assert_grads(grads, want, bf, f"bf16 Nq{Nq} Nk{Nk} D{D}")


def test_scale_values(device):
    """Non-default, negative and zero softmax scales."""
    q, k, v = seeded((1, 2, 96, 64), 9), seeded((1, 2, 96, 64), 10), seeded((1, 2, 96, 64), 11)
    do = seeded((1, 2, 96, 64), 12)
    for scale in (0.3, -0.125, 0.0):
        print(f"[bwd scale] {scale}", flush=True)
        grads = run_backward(q, k, v, do, True, device, scale=scale)
        want = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), causal=1, scale=scale)
        assert_grads(grads, want, torch.float16, f"scale {scale}")


def test_autograd_function(device):
    """flash_attention under autograd: its gradients are the backward op's,
    and the reference-named forward keeps its forward-only contract."""
    print("[bwd autograd]", flush=True)
    B, Hq, Hkv, N, D = 2, 8, 2, 300, 128
    q, k, v = seeded((B, Hq, N, D), 13), seeded((B, Hkv, N, D), 14), seeded((B, Hkv, N, D), 15)
    do = seeded((B, Hq, N, D), 16)
    leaves = [t.to(device).requires_grad_() for t in (q, k, v)]
    o = flash_attention(*leaves, causal=True)
    o.backward(do.to(device))
    direct = run_backward(q, k, v, do, True, device)
    for leaf, d in zip(leaves, direct):
        assert torch.equal(leaf.grad, d)
    want = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), causal=1)
    assert_grads([l.grad for l in leaves], want, torch.float16, "autograd")
    # no double backward through the kernels
    leaves2 = [t.to(device).requires_grad_() for t in (q, k, v)]
    gq, = torch.autograd.grad(flash_attention(*leaves2, causal=True).float().square().sum(),
                              leaves2[0], create_graph=True)
    with pytest.raises(RuntimeError):
        gq.sum().backward()
    # the reference's Function still raises in backward (reference tests/test_api.py:38)
    x = [t.to(device).requires_grad_() for t in (q, k, v)]
    with pytest.raises(NotImplementedError, match="Backward pass is not implemented"):
        flash_attention_forward(*x, causal=True).sum().backward()


def test_deterministic_and_strided(device):
    """Bitwise-repeatable; strided [B, N, H, D] views give the same gradients."""
    print("[bwd strided]", flush=True)
    B, Hq, Hkv, N, D = 2, 8, 4, 257, 64
    q, k, v = seeded((B, Hq, N, D), 17), seeded((B, Hkv, N, D), 18), seeded((B, Hkv, N, D), 19)
    do = seeded((B, Hq, N, D), 20)
    a = run_backward(q, k, v, do, True, device)
    b = run_backward(q, k, v, do, True, device)
    for x, y in zip(a, b):
        assert torch.equal(x, y)
    views = [t.to(device).transpose(1, 2).contiguous().transpose(1, 2) for t in (q, k, v, do)]
    assert not views[0].is_contiguous()
    o, lse = flash_attention_forward_ex(*views[:3], causal=True, return_lse=True)
    c = flash_attention_backward(views[3], *views[:3], o, lse, causal=True)
    torch.cuda.synchronize()
    for x, y in zip(a, c):
        assert torch.equal(x, y)


@pytest.mark.parametrize("B,Hq,Hkv,N,causal", [(1, 16, 4, 4096, False), (1, 16, 4, 4096, True),
                                               (2, 64, 8, 16384, True)])
def test_key_sum_identities_at_size(device, B, Hq, Hkv, N, causal):
    """At sizes the oracle cannot reach (up to the C5 shape, 268M elements per
    Q-shaped tensor): sum_j dK_j = 0 and sum_j dV_j equals the group's sum of
    dO rows, within the rounding of the fp16 gradients."""
    print(f"[bwd identities] B={B} Hq={Hq} Hkv={Hkv} N={N} causal={causal}", flush=True)
    D = 128
    g = torch.Generator(device).manual_seed(21)
    q, k, v, do = (torch.randn(s, generator=g, device=device).half()
                   for s in ((B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)))
    dq, dk, dv = run_backward(q, k, v, do, causal, device)
    dk, dv = dk.double(), dv.double()
    r_k = (dk.sum(2).abs().amax() / dk.abs().sum(2).amax()).item()
    do_g = do.double().reshape(B, Hkv, Hq // Hkv, N, D).sum(dim=(2, 3))
    r_v = ((dv.sum(2) - do_g).abs().amax() / dv.abs().sum(2).amax()).item()
    print(f"  sum dK residual {r_k:.2e}, sum dV residual {r_v:.2e}", flush=True)
    assert r_k < 2e-3 and r_v < 2e-3
    assert torch.isfinite(dq).all()


def test_empty_and_degenerate(device):
    """No query rows: dK = dV = 0; zero batch: empty gradients."""
    print("[bwd empty]", flush=True)
    k = seeded((1, 2, 50, 64), 25).to(device)
    q = torch.empty(1, 4, 0, 64, dtype=torch.float16, device=device)
    o = torch.empty_like(q)
    lse = torch.empty(1, 4, 0, dtype=torch.float32, device=device)
    dq, dk, dv = _C.flash_attention_backward(o, q, k, k, o, lse, 0, 0.125)
    torch.cuda.synchronize()
    assert dq.shape == q.shape and torch.count_nonzero(dk) == 0 and torch.count_nonzero(dv) == 0
    z = torch.empty(0, 2, 8, 64, dtype=torch.float16, device=device)
    out = _C.flash_attention_backward(z, z, z, z, z, torch.empty(0, 2, 8, device=device), 1, 0.1)
    assert all(t.numel() == 0 for t in out)


@pytest.mark.parametrize("masked", [False, True])
def test_graph_capture_replays(device, masked):
    """The backward captured in a HIP graph (three kernel launches, workspace
    from the graph's pool, no memsets; with a mask also the packing kernel
    and the masked forward) and replayed three times with fresh inputs and
    eager work in between: every replay bitwise equal to eager."""
    print(f"[bwd graph] masked={masked}", flush=True)
    B, Hq, Hkv, N, D = 1, 8, 2, 700, 128
    q, k, v, do = (torch.empty(s, dtype=torch.float16, device=device)
                   for s in ((B, Hq, N, D), (B, Hkv, N, D), (B, Hkv, N, D), (B, Hq, N, D)))
    mask = None
    if masked:
        g = torch.Generator("cpu").manual_seed(70)
        mask = (torch.rand(B, 1, N, N, generator=g) < 0.8).to(device)

    def fill(seed):
        for i, t in enumerate((q, k, v, do)):
            t.copy_(seeded(t.shape, seed + i))

    def call():
        o, lse = flash_attention_forward_ex(q, k, v, causal=True, return_lse=True,
                                            attn_mask=mask)
        return flash_attention_backward(do, q, k, v, o, lse, causal=True, attn_mask=mask)

    fill(30)
    side = torch.cuda.Stream(device)
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(2):
            call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = call()
    for rep in range(3):
        fill(40 + 10 * rep)
        graph.replay()
        junk = torch.randn(1 << 20, device=device).sum()
        torch.cuda.synchronize()
        expect = call()
        torch.cuda.synchronize()
        assert torch.isfinite(junk)
        for x, y in zip(outs, expect):
            assert torch.equal(x, y), rep


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal,mshape", [
    (2, 4, 2, 200, 200, 128, False, "b1qk"),
    (1, 4, 4, 150, 300, 64, True, "bhqk"),
    (2, 8, 2, 333, 333, 128, "bottom_right", "qk"),
    (1, 2, 1, 257, 129, 64, False, "b1qk"),
    # key padding broadcast over heads and rows (mask row stride 0)
    (2, 4, 2, 180, 260, 64, True, "b11k"),
    (2, 8, 4, 300, 300, 128, "bottom_right", "b11k"),
])
def test_backward_with_mask(device, dtype, B, Hq, Hkv, Nq, Nk, D, causal, mshape):
    """Boolean attn_mask (broadcast over batch/heads/rows as given), combined
    with the causal modes, including rows that see no key; through the
    autograd Function."""
    print(f"[bwd mask] {dtype} B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} "
          f"causal={causal} mask={mshape}", flush=True)
    shape = {"b1qk": (B, 1, Nq, Nk), "bhqk": (B, Hq, Nq, Nk), "qk": (Nq, Nk),
             "b11k": (B, 1, 1, Nk)}[mshape]
    g = torch.Generator("cpu").manual_seed(50)
    mask = torch.rand(*shape, generator=g) < 0.7
    padding = mshape == "b11k"
    if padding:
        mask[0, ..., Nk - 40:] = False  # batch 0 right-padded by 40 keys
    else:
        mask[..., 5, :] = False  # a row that sees no key
    q, k, v = seeded((B, Hq, Nq, D), 51, dtype), seeded((B, Hkv, Nk, D), 52, dtype), \
        seeded((B, Hkv, Nk, D), 53, dtype)
    do = seeded((B, Hq, Nq, D), 54, dtype)
    leaves = [t.to(device).requires_grad_() for t in (q, k, v)]
    o = flash_attention(*leaves, causal=causal, attn_mask=mask.to(device))
    o.backward(do.to(device))
    torch.cuda.synchronize()
    want = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), causal=CODE[causal],
                                      attn_mask=mask.numpy())
    if not padding:
        assert torch.count_nonzero(leaves[0].grad[:, :, 5]) == 0
    else:  # keys hidden from every row get no gradient
        assert torch.count_nonzero(leaves[1].grad[0, :, Nk - 40:]) == 0
        assert torch.count_nonzero(leaves[2].grad[0, :, Nk - 40:]) == 0
    assert_grads([l.grad for l in leaves], want, dtype, f"mask {mshape}")


def test_side_stream(device):
    """The backward runs on the caller's current stream (its workspace comes
    from that stream's pool): a call on a side stream, with the default
    stream busy, gives bitwise the same gradients."""
    print("[bwd side stream]", flush=True)
    B, Hq, Hkv, N, D = 2, 8, 2, 500, 128
    q, k, v = seeded((B, Hq, N, D), 60), seeded((B, Hkv, N, D), 61), seeded((B, Hkv, N, D), 62)
    do = seeded((B, Hq, N, D), 63)
    want = run_backward(q, k, v, do, True, device)
    qd, kd, vd, dod = (t.to(device) for t in (q, k, v, do))
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device)
    busy = torch.randn(4096, 4096, device=device)
    with torch.cuda.stream(side):
        o, lse = flash_attention_forward_ex(qd, kd, vd, causal=True, return_lse=True)
        got = flash_attention_backward(dod, qd, kd, vd, o, lse, causal=True)
    for _ in range(4):
        busy = busy @ busy * 1e-3  # default-stream work meanwhile
    torch.cuda.synchronize()
    for x, y in zip(want, got):
        assert torch.equal(x, y)


def per_head_mask(B, Hq, N, seed):
    """[B, Hq, N, N] boolean mask that differs between the query heads of a
    KV group: head h sees a causal sliding window of its own width (one head
    the whole causal prefix), a tenth of the window's keys dropped at
    random, and a block of rows of every odd head sees no key at all.  The
    dK/dV kernel then has to take the union of the rows' key spans over the
    group's heads to find the query tiles of its key block."""
    g = torch.Generator("cpu").manual_seed(seed)
    i = torch.arange(N)
    m = torch.zeros(B, Hq, N, N, dtype=torch.bool)
    for h in range(Hq):
        w = [N, 37, 150, 400][h % 4] + 13 * (h // 4)
        band = (i[None, :] <= i[:, None]) & (i[None, :] > i[:, None] - w)
        for b in range(B):
            keep = torch.rand(N, N, generator=g) >= 0.1
            m[b, h] = band & keep
            if h % 2 == 1:
                r0 = (97 * (h + b)) % (N - 80)
                m[b, h, r0:r0 + 70] = False
    return m


def split_mask(B, N):
    """[B, 1, N, N] mask whose rows alternate between two disjoint key spans:
    even rows see the first 96 keys, odd rows the last 96.  Every 64-row query
    tile's span (the union over its rows) then covers all keys although no
    row sees a key in between, so the dK/dV kernel keeps query tiles that
    contribute nothing to its key blocks there."""
    i = torch.arange(N)
    even = (i[:, None] % 2 == 0) & (i[None, :] < 96)
    odd = (i[:, None] % 2 == 1) & (i[None, :] >= N - 96)
    return (even | odd)[None, None].expand(B, 1, N, N).clone()


@pytest.mark.parametrize("B,Hq,Hkv,N,D,bf16,kind",
                         [(3, 4, 2, 700, 64, False, "padded"), (2, 8, 2, 1100, 128, True, "padded"),
                          (2, 8, 2, 600, 64, False, "per_head"), (1, 6, 2, 900, 128, False, "per_head"),
                          (2, 4, 2, 640, 64, False, "split"), (1, 4, 1, 520, 128, True, "split")])
def test_backward_mask_ranges_bitwise(device, B, Hq, Hkv, N, D, bf16, kind):
    """Through the C ABI: a mask given as bits, with and without mask_ranges:
    dQ, dK and dV bit for bit the same (the skipped key tiles of dQ and query
    tiles of dK/dV see nothing of each other), and within the bar of the
    float64 closed form.  The mask is a causal one with left padding shared
    by every head ("padded"), a [B, Hq, N, N] mask whose rows' spans differ
    between the query heads of a group and some of whose rows see no key
    ("per_head"), or rows alternating between two disjoint key spans
    ("split", split_mask)."""
    per_head = kind == "per_head"
    import ctypes
    from capi_types import LIB, BwdParams
    print(f"[bwd ranges] B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} bf16={bf16} kind={kind}", flush=True)
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_backward.argtypes = [ctypes.POINTER(BwdParams)]
    lib.fa_sm75_backward_workspace_size.argtypes = [ctypes.POINTER(BwdParams)]
    lib.fa_sm75_backward_workspace_size.restype = ctypes.c_int64
    lib.fa_sm75_set_contiguous_bwd_strides.argtypes = [ctypes.POINTER(BwdParams)]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    pk = lib.fa_sm75_pack_mask_ranges
    pk.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p] * 3
    dt = torch.bfloat16 if bf16 else torch.float16
    g = torch.Generator("cpu").manual_seed(N + D)
    q, k, v, do = (torch.randn(B, h, N, D, generator=g).to(dt) for h in (Hq, Hkv, Hkv, Hq))
    if per_head:
        m = per_head_mask(B, Hq, N, N + D)
    elif kind == "split":
        m = split_mask(B, N)
    else:
        i = torch.arange(N)
        m = (i[None, :] <= i[:, None])[None, None].expand(B, 1, N, N).clone()
        for b in range(B):
            m[b, :, :, : (b * N) // (2 * B)] = False
    mh = m.size(1)
    qd, kd, vd, dod, md = (t.to(device) for t in (q, k, v, do, m))
    o, lse = flash_attention_forward_ex(qd, kd, vd, attn_mask=md, return_lse=True)
    words = (N + 63) // 64
    bits = torch.empty(B, mh, N, words, dtype=torch.int64, device=device)
    rng = torch.empty(B, mh, N, 2, dtype=torch.int32, device=device)
    stream = torch.cuda.current_stream().cuda_stream
    st = md.stride()
    assert pk(md.data_ptr(), B, mh, N, N, st[0], st[1] if mh > 1 else 0, st[2], st[3],
              bits.data_ptr(), rng.data_ptr(), stream) == 0
    if per_head:  # some rows see nothing: their range is empty
        assert (rng[..., 0] >= rng[..., 1]).any().item()

    def run(with_ranges):
        dq, dk, dv = torch.empty_like(qd), torch.empty_like(kd), torch.empty_like(vd)
        p = BwdParams()
        p.q, p.k, p.v, p.o, p.dout, p.lse, p.dq, p.dk, p.dv = (
            t.data_ptr() for t in (qd, kd, vd, o, dod, lse, dq, dk, dv))
        p.batch, p.heads_q, p.heads_kv, p.seq_len, p.seq_len_kv, p.head_dim = B, Hq, Hkv, N, N, D
        lib.fa_sm75_set_contiguous_bwd_strides(ctypes.byref(p))
        p.scale, p.dtype, p.stream = D ** -0.5, 1 if bf16 else 0, stream
        p.mask_bits, p.mask_stride_b, p.mask_stride_q = bits.data_ptr(), mh * N * words, words
        p.mask_stride_h = N * words if mh > 1 else 0
        if with_ranges:
            p.mask_ranges, p.mask_ranges_stride_b, p.mask_ranges_stride_q = rng.data_ptr(), mh * N, 1
            p.mask_ranges_stride_h = N if mh > 1 else 0
        n = lib.fa_sm75_backward_workspace_size(ctypes.byref(p))
        ws = torch.empty(n, dtype=torch.uint8, device=device)
        p.workspace, p.workspace_bytes = ws.data_ptr(), n
        assert lib.fa_sm75_backward(ctypes.byref(p)) == 0, lib.fa_sm75_last_error()
        torch.cuda.synchronize()
        return dq, dk, dv

    with_r = run(True)
    without = run(False)
    for a_, b_ in zip(with_r, without):
        assert torch.equal(a_, b_)
    npf = lambda t: t.float().cpu().numpy()
    wants = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), attn_mask=m.numpy(),
                                       delta_from_o=npf(o))
    ba, br = (1e-2, 4e-2) if bf16 else (2e-3, 1e-2)
    for name, gt, w in zip(("dQ", "dK", "dV"), with_r, wants):
        gg = npf(gt).astype(np.float64)
        sc = max(float(np.abs(w).max()), 1e-2)
        worst = float((np.abs(gg - w) / (ba * sc + br * np.abs(w) + 1e-30)).max())
        print(f"  {name}: worst/bar={worst:.3f}", flush=True)
        assert worst <= 1.0, (name, worst)
