"""Pins the backward oracle (oracle.attention_ref.attention_backward_f64).

The oracle restates the gradient of the reference's attention math in closed
form.  It is checked against things that do not retype that formula:
  * torch.autograd through torch's own matmul/softmax, in float64 on the CPU
    (an independent derivation of the same gradient);
  * central finite differences of L = sum(O * dO) (the definition of the
    gradient), on tiny inputs;
  * two invariants of softmax attention: the keys' dK rows sum to zero
    (each row of dS sums to zero), and the keys' dV rows sum to the dO rows
    of the queries that see at least one key (each row of P sums to one);
  * planted mistakes (in the oracle's math, on the CPU) that must fail them.
"""
import numpy as np
import pytest
import torch

from oracle import attention_ref as ref


def rnd(shape, seed):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float16)


def torch_grads(q, k, v, do, causal, scale, attn_mask=None):
    """float64 autograd through torch's ops, GQA by repeat_interleave."""
    Q = torch.tensor(q.astype(np.float64), requires_grad=True)
    K = torch.tensor(k.astype(np.float64), requires_grad=True)
    V = torch.tensor(v.astype(np.float64), requires_grad=True)
    g = Q.shape[1] // K.shape[1]
    Ke, Ve = K.repeat_interleave(g, 1), V.repeat_interleave(g, 1)
    S = Q @ Ke.transpose(-1, -2) * scale
    mask = ref.causal_mask(q.shape[2], k.shape[2], causal)
    if mask is not None:
        S = S.masked_fill(torch.tensor(mask), float("-inf"))
    if attn_mask is not None:
        S = S.masked_fill(~torch.tensor(attn_mask), float("-inf"))
    P = torch.softmax(S, -1).nan_to_num(0.0)
    O = P @ Ve
    O.backward(torch.tensor(do.astype(np.float64)))
    return Q.grad.numpy(), K.grad.numpy(), V.grad.numpy()


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal
    (1, 1, 1, 5, 5, 64, False),
    (1, 2, 2, 17, 17, 64, True),
    (2, 4, 2, 9, 9, 128, True),
    (1, 4, 1, 6, 11, 64, "bottom_right"),
    (1, 2, 1, 12, 5, 64, "bottom_right"),   # rows that see no key
    (1, 3, 1, 7, 13, 128, True),            # top-left with Nq < Nk
]
CODE = {False: 0, True: 1, "bottom_right": 2}


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", CASES)
def test_matches_torch_autograd(B, Hq, Hkv, Nq, Nk, D, causal):
    q, k, v = rnd((B, Hq, Nq, D), 1), rnd((B, Hkv, Nk, D), 2), rnd((B, Hkv, Nk, D), 3)
    do = rnd((B, Hq, Nq, D), 4)
    c = CODE[causal]
    got = ref.attention_backward_f64(q, k, v, do, causal=c)
    want = torch_grads(q, k, v, do, c, ref.default_scale(D))
    for name, g, w in zip(("dQ", "dK", "dV"), got, want):
        np.testing.assert_allclose(g, w, rtol=1e-9, atol=1e-11, err_msg=name)


def test_finite_differences():
    """dL/dx for L = sum(O * dO), by central differences in float64."""
    B, Hq, Hkv, N, D = 1, 2, 1, 6, 64
    rng = np.random.default_rng(7)
    q = rng.standard_normal((B, Hq, N, D))
    k = rng.standard_normal((B, Hkv, N, D))
    v = rng.standard_normal((B, Hkv, N, D))
    do = rng.standard_normal((B, Hq, N, D))
    for causal in (0, 1):
        grads = ref.attention_backward_f64(q, k, v, do, causal=causal)

        def loss(qq, kk, vv):
            return float((ref.attention_f64(qq, kk, vv, causal=causal) * do).sum())

        h = 1e-6
        for which, g in enumerate(grads):
            for _ in range(6):
                idx = tuple(int(rng.integers(0, s)) for s in (q, k, v)[which].shape)
                args = [q.copy(), k.copy(), v.copy()]
                args[which][idx] += h
                up = loss(*args)
                args[which][idx] -= 2 * h
                dn = loss(*args)
                fd = (up - dn) / (2 * h)
                assert abs(fd - g[idx]) <= 1e-6 * (1 + abs(fd)), (causal, which, idx, fd, g[idx])


def key_sum_residuals(q, k, v, do, causal, grads):
    """max |sum_j dK_j| / sum_j |dK_j| and the same for sum_j dV_j minus the
    dO rows that see a key (per KV head, over its group)."""
    dq, dk, dv = grads
    B, Hq, N, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    g = Hq // Hkv
    mask = ref.causal_mask(N, Nk, causal)
    sees = np.ones(N, bool) if mask is None else ~mask.all(axis=1)
    dk_sum = dk.sum(axis=2)
    r_k = np.abs(dk_sum).max() / np.abs(dk).sum(axis=2).max()
    do_rows = (do.astype(np.float64) * sees[None, None, :, None]).reshape(B, Hkv, g, N, D)
    r_v = np.abs(dv.sum(axis=2) - do_rows.sum(axis=(2, 3))).max() / np.abs(dv).sum(axis=2).max()
    return r_k, r_v


@pytest.mark.parametrize("causal", [0, 1, 2])
def test_key_sum_invariants(causal):
    q, k, v = rnd((2, 4, 20, 64), 11), rnd((2, 2, 30, 64), 12), rnd((2, 2, 30, 64), 13)
    do = rnd((2, 4, 20, 64), 14)
    grads = ref.attention_backward_f64(q, k, v, do, causal=causal)
    r_k, r_v = key_sum_residuals(q, k, v, do, causal, grads)
    assert r_k < 1e-12 and r_v < 1e-12, (r_k, r_v)


PLANTS = ["no_rowsum", "transposed_p", "no_scale_dk", "wrong_gqa_sum"]


def planted_backward(kind, q, k, v, do, causal):
    """The oracle's math with one plausible mistake."""
    B, Hq, N, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    g = Hq // Hkv
    ke, ve = ref.expand_kv_for_gqa(q, k, v)
    qf, kf, vf, dof = (x.astype(np.float64) for x in (q, ke, ve, do))
    s = ref.default_scale(D)
    S = qf @ np.swapaxes(kf, -1, -2) * s
    mask = ref.causal_mask(N, Nk, causal)
    if mask is not None:
        S[..., mask] = -np.inf
    P = np.exp(S - S.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    dv = (P if kind == "transposed_p" else np.swapaxes(P, -1, -2)) @ dof
    dP = dof @ np.swapaxes(vf, -1, -2)
    dS = P * dP if kind == "no_rowsum" else P * (dP - (dP * P).sum(-1, keepdims=True))
    dq = s * dS @ kf
    dk = (1.0 if kind == "no_scale_dk" else s) * np.swapaxes(dS, -1, -2) @ qf
    if kind == "wrong_gqa_sum":
        dk = dk.reshape(B, g, Hkv, Nk, D).sum(axis=1)
        dv = dv.reshape(B, g, Hkv, Nk, D).sum(axis=1)
    else:
        dk = dk.reshape(B, Hkv, g, Nk, D).sum(axis=2)
        dv = dv.reshape(B, Hkv, g, Nk, D).sum(axis=2)
    return dq, dk, dv


@pytest.mark.parametrize("kind", PLANTS)
def test_planted_mistakes_are_detected(kind):
    """Each plant must fail the autograd comparison or an invariant."""
    q, k, v = rnd((1, 4, 16, 64), 21), rnd((1, 2, 16, 64), 22), rnd((1, 2, 16, 64), 23)
    do = rnd((1, 4, 16, 64), 24)
    bad = planted_backward(kind, q, k, v, do, 1)
    want = torch_grads(q, k, v, do, 1, ref.default_scale(64))
    differs = any(not np.allclose(b, w, rtol=1e-6, atol=1e-8) for b, w in zip(bad, want))
    r_k, r_v = key_sum_residuals(q, k, v, do, 1, bad)
    assert differs or r_k > 1e-6 or r_v > 1e-6
    # and the unplanted oracle passes the same checks
    good = ref.attention_backward_f64(q, k, v, do, causal=1)
    assert all(np.allclose(b, w, rtol=1e-9, atol=1e-11) for b, w in zip(good, want))


@pytest.mark.parametrize("mshape,causal", [((2, 1, 9, 14), 0), ((1, 4, 9, 14), 1),
                                           ((9, 14), 2), ((2, 4, 1, 14), 0)])
def test_masked_matches_torch_autograd(mshape, causal):
    """Boolean masks (broadcast shapes, combined with each causal mode, rows
    that see no key) against autograd with the same masked_fill."""
    q, k, v = rnd((2, 4, 9, 64), 31), rnd((2, 2, 14, 64), 32), rnd((2, 2, 14, 64), 33)
    do = rnd((2, 4, 9, 64), 34)
    mask = np.random.default_rng(35).random(mshape) < 0.6
    if len(mshape) == 4 and mshape[2] > 1:
        mask[..., 3, :] = False  # a row that sees no key
    got = ref.attention_backward_f64(q, k, v, do, causal=causal, attn_mask=mask)
    want = torch_grads(q, k, v, do, causal, ref.default_scale(64), attn_mask=mask)
    for name, g, w in zip(("dQ", "dK", "dV"), got, want):
        np.testing.assert_allclose(g, w, rtol=1e-9, atol=1e-11, err_msg=name)


@pytest.mark.parametrize("causal", [False, True, "bottom_right"])
def test_delta_from_o(causal):
    """delta_from_o: with the exact O the row term rowsum(dO o O) equals
    rowsum(dP o P), so the gradients are unchanged; with O + E every query
    row i moves by -rowsum(dO_i o E_i) P_i in dS, so dQ and dK shift by that
    term's products with K and Q (P from torch in float64) and dV not at all."""
    B, Hq, Hkv, Nq, Nk, D = 1, 4, 2, 7, 11, 64
    q, k, v = rnd((B, Hq, Nq, D), 21), rnd((B, Hkv, Nk, D), 22), rnd((B, Hkv, Nk, D), 23)
    do = rnd((B, Hq, Nq, D), 24)
    c = CODE[causal]
    scale = ref.default_scale(D)
    base = ref.attention_backward_f64(q, k, v, do, causal=c)
    o = ref.attention_f64(q, k, v, causal=c)
    same = ref.attention_backward_f64(q, k, v, do, causal=c, delta_from_o=o)
    for g, w in zip(same, base):
        np.testing.assert_allclose(g, w, rtol=1e-10, atol=1e-12)
    e = np.random.default_rng(25).standard_normal(o.shape) * 1e-2
    moved = ref.attention_backward_f64(q, k, v, do, causal=c, delta_from_o=o + e)
    g = Hq // Hkv
    K = torch.tensor(k.astype(np.float64)).repeat_interleave(g, 1)
    Q = torch.tensor(q.astype(np.float64))
    S = Q @ K.transpose(-1, -2) * scale
    m = ref.causal_mask(Nq, Nk, c)
    if m is not None:
        S = S.masked_fill(torch.tensor(m), float("-inf"))
    P = torch.softmax(S, -1).nan_to_num(0.0)
    shift = -(torch.tensor(do.astype(np.float64)) * torch.tensor(e)).sum(-1, keepdim=True) * P
    want_dq = base[0] + scale * (shift @ K).numpy()
    want_dk = base[1] + scale * (shift.transpose(-1, -2) @ Q).numpy().reshape(B, Hkv, g, Nk, D).sum(2)
    np.testing.assert_allclose(moved[0], want_dq, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(moved[1], want_dk, rtol=1e-9, atol=1e-11)
    np.testing.assert_allclose(moved[2], base[2], rtol=0, atol=0)
