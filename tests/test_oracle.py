"""Pins the CPU oracle before it is trusted as the parity checker.

Each oracle function is checked against something that does not retype its
own formula:
  * the long-double C statement (oracle/attention_oracle.c), a different
    language, precision and loop structure;
  * closed forms / invariants of softmax attention that a dropped term,
    flipped mask, wrong scale or transposed operand would break;
  * planted mistakes (in the oracle, on the CPU) that those checks must catch;
  * the reference's own known-answer inputs (glibc rand() streams).
"""
import numpy as np
import pytest

from oracle import attention_ref as ref
from oracle import c_oracle


def rnd(shape, seed, std=1.0):
    r = np.random.default_rng(seed)
    return (r.standard_normal(shape) * std).astype(np.float16)


SHAPES = [
    # B, Hq, Hkv, N, D, causal
    (1, 1, 1, 1, 64, False),
    (1, 1, 1, 1, 64, True),
    (1, 2, 2, 16, 64, True),
    (2, 2, 2, 17, 128, False),
    (1, 4, 1, 33, 64, True),
    (1, 8, 2, 40, 128, True),
    (1, 2, 2, 127, 64, False),
]


@pytest.mark.parametrize("B,Hq,Hkv,N,D,causal", SHAPES)
def test_numpy_matches_long_double(B, Hq, Hkv, N, D, causal):
    q = rnd((B, Hq, N, D), 1)
    k = rnd((B, Hkv, N, D), 2)
    v = rnd((B, Hkv, N, D), 3)
    o32 = ref.attention_reference(q, k, v, causal=causal, return_f32=True)
    o_ld, lse_ld = c_oracle.attention_ld(q, k, v, causal=causal)
    # fp32 evaluation of the same closed form: ~1e-6 agreement
    np.testing.assert_allclose(o32, o_ld, rtol=0, atol=2e-5)
    # fp16 output: the fp32 value (error < 2e-6 absolute, from cancellation in
    # P V) rounded to fp16 (at most half an ulp = |x| 2^-11)
    o16 = ref.attention_reference(q, k, v, causal=causal)
    assert np.all(np.abs(o16.astype(np.float64) - o_ld) <= np.abs(o_ld) * 2 ** -10 + 2e-6)
    # fp64 brute force in numpy agrees with C long double to rounding
    np.testing.assert_allclose(ref.attention_f64(q, k, v, causal=causal), o_ld, atol=1e-12)
    lse = ref.attention_lse(q, k, causal=causal)
    np.testing.assert_allclose(lse, lse_ld, atol=1e-10)


def test_chunked_equals_full():
    q = rnd((2, 4, 300, 64), 4)
    k = rnd((2, 2, 300, 64), 5)
    v = rnd((2, 2, 300, 64), 6)
    for causal in (False, True):
        full = ref.attention_reference(q, k, v, causal=causal, return_f32=True)
        ch = ref.attention_reference_chunked(q, k, v, causal=causal, rows=64, return_f32=True)
        np.testing.assert_allclose(ch, full, atol=2e-6, rtol=0)
        sub = ref.attention_reference_chunked(q, k, v, causal=causal, rows=128, heads=[3, 1],
                                              return_f32=True)
        np.testing.assert_allclose(sub, full[:, [3, 1]], atol=2e-6, rtol=0)


def test_torch_cpu_restatement_matches_numpy():
    import torch

    q = rnd((1, 4, 257, 128), 7)
    k = rnd((1, 1, 257, 128), 8)
    v = rnd((1, 1, 257, 128), 9)
    for causal in (False, True):
        a = ref.attention_reference(q, k, v, causal=causal).astype(np.float32)
        b = ref.attention_reference_torch_cpu(torch.from_numpy(q), torch.from_numpy(k),
                                              torch.from_numpy(v), causal=causal,
                                              rows=100).float().numpy()
        # both round the same fp32 value to fp16: at most one ulp apart
        assert np.all(np.abs(a - b) <= np.abs(a) * 2 ** -10 + 2 ** -24)
        # unrounded, and with a causal block's hidden keys skipped: the fp32
        # values agree to summation order
        a32 = ref.attention_reference(q, k, v, causal=causal, return_f32=True)
        for skip in (False, True):
            b32 = ref.attention_reference_torch_cpu(
                torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), causal=causal,
                rows=100, heads=[2, 0], return_f32=True, skip_hidden=skip)
            assert b32.dtype == torch.float32
            np.testing.assert_allclose(b32.numpy(), a32[:, [2, 0]], atol=2e-6, rtol=0)


# ---- invariants (closed forms) ---------------------------------------------

def test_causal_row0_is_v0():
    q, k, v = rnd((1, 2, 50, 64), 10), rnd((1, 2, 50, 64), 11), rnd((1, 2, 50, 64), 12)
    o = ref.attention_reference(q, k, v, causal=True)
    np.testing.assert_array_equal(o[:, :, 0], v[:, :, 0])


def test_constant_v_gives_v():
    q, k = rnd((1, 1, 40, 64), 13), rnd((1, 1, 40, 64), 14)
    v = np.full((1, 1, 40, 64), 0.375, dtype=np.float16)
    for causal in (False, True):
        o = ref.attention_reference(q, k, v, causal=causal, return_f32=True)
        np.testing.assert_allclose(o, 0.375, atol=1e-6)


def test_key_permutation_invariance():
    q, k, v = rnd((1, 1, 64, 64), 15), rnd((1, 1, 64, 64), 16), rnd((1, 1, 64, 64), 17)
    perm = np.random.default_rng(0).permutation(64)
    a = ref.attention_reference(q, k, v, return_f32=True)
    b = ref.attention_reference(q, k[:, :, perm], v[:, :, perm], return_f32=True)
    np.testing.assert_allclose(a, b, atol=2e-6)


def test_zero_scale_is_prefix_mean():
    q, k, v = rnd((1, 1, 30, 64), 18), rnd((1, 1, 30, 64), 19), rnd((1, 1, 30, 64), 20)
    o = ref.attention_reference(q, k, v, causal=True, scale=0.0, return_f32=True)
    vf = v.astype(np.float64)[0, 0]
    expect = np.cumsum(vf, axis=0) / np.arange(1, 31)[:, None]
    np.testing.assert_allclose(o[0, 0], expect, atol=1e-5)
    o_full = ref.attention_reference(q, k, v, causal=False, scale=0.0, return_f32=True)
    np.testing.assert_allclose(o_full[0, 0], np.broadcast_to(vf.mean(0), (30, 64)), atol=1e-5)


def test_single_key_gives_v():
    q, k, v = rnd((2, 3, 1, 128), 21), rnd((2, 3, 1, 128), 22), rnd((2, 3, 1, 128), 23)
    np.testing.assert_array_equal(ref.attention_reference(q, k, v), v)


def test_gqa_equals_explicit_repeat():
    q, k, v = rnd((1, 8, 20, 64), 24), rnd((1, 2, 20, 64), 25), rnd((1, 2, 20, 64), 26)
    a = ref.attention_reference(q, k, v, causal=True)
    b = ref.attention_reference(q, np.repeat(k, 4, axis=1), np.repeat(v, 4, axis=1), causal=True)
    np.testing.assert_array_equal(a, b)
    # head h reads KV head h // 4 (not h % 2)
    h = 5
    one = ref.attention_reference(q[:, h:h + 1], k[:, 1:2], v[:, 1:2], causal=True)
    np.testing.assert_array_equal(a[:, h:h + 1], one)
    with pytest.raises(RuntimeError, match="not divisible"):
        ref.expand_kv_for_gqa(q, rnd((1, 3, 20, 64), 1), rnd((1, 3, 20, 64), 2))


def test_lse_closed_form():
    from scipy.special import logsumexp

    q, k = rnd((1, 2, 25, 64), 27), rnd((1, 2, 25, 64), 28)
    S = (q.astype(np.float64) @ np.swapaxes(k.astype(np.float64), -1, -2)) / 8.0
    S_c = S.copy()
    S_c[..., np.triu(np.ones((25, 25), bool), 1)] = -np.inf
    np.testing.assert_allclose(ref.attention_lse(q, k, causal=False), logsumexp(S, -1), atol=1e-12)
    np.testing.assert_allclose(ref.attention_lse(q, k, causal=True), logsumexp(S_c, -1), atol=1e-12)


# ---- the reference scalar kernel's order (online softmax) -------------------

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("tile", [32, 64])
def test_online_order_matches_closed_form(causal, tile):
    q, k, v = rnd((1, 2, 100, 64), 29), rnd((1, 2, 100, 64), 30), rnd((1, 2, 100, 64), 31)
    o_ld, _ = c_oracle.attention_ld(q, k, v, causal=causal)
    o = c_oracle.online_f32(q, k, v, causal=causal, tile=tile)
    np.testing.assert_allclose(o, o_ld, atol=2e-5)
    # rounding P to fp16 before PV (what the MFMA kernels do) stays well
    # inside the 2e-3 parity tolerance
    o_rp = c_oracle.online_f32(q, k, v, causal=causal, tile=tile, round_p=True)
    assert np.abs(o_rp - o_ld).max() < 5e-4


# ---- planted mistakes must be caught ----------------------------------------

def _planted(kind, q, k, v, causal):
    qf, kf, vf = (x.astype(np.float32) for x in (q, k, v))
    scale = 1.0 / np.sqrt(q.shape[-1])
    n = q.shape[-2]
    if kind == "no_scale":
        S = qf @ np.swapaxes(kf, -1, -2)
    elif kind == "transposed_scores":
        S = (kf @ np.swapaxes(qf, -1, -2)) * scale
    else:
        S = (qf @ np.swapaxes(kf, -1, -2)) * scale
    if causal:
        tri = np.triu(np.ones((n, n), bool), 1)
        S[..., tri.T if kind == "mask_flipped" else tri] = -np.inf
    if kind == "mask_diag_excluded" and causal:
        S[..., np.eye(n, dtype=bool)] = -np.inf
        S[..., 0, 0] = 0.0
    P = np.exp(S - S.max(-1, keepdims=True))
    P /= P.sum(-1, keepdims=True)
    if kind == "v_transposed_rows":
        vf = vf[..., ::-1, :]
    return P @ vf


@pytest.mark.parametrize("kind", ["no_scale", "transposed_scores", "mask_flipped",
                                  "mask_diag_excluded", "v_transposed_rows"])
def test_planted_mistakes_are_detected(kind):
    q, k, v = rnd((1, 1, 48, 64), 32), rnd((1, 1, 48, 64), 33), rnd((1, 1, 48, 64), 34)
    causal = kind.startswith("mask") or kind == "transposed_scores"
    bad = _planted(kind, q, k, v, causal)
    good, _ = c_oracle.attention_ld(q, k, v, causal=causal)
    res = ref.check_correctness(bad, good, atol=2e-3, rtol=1e-2)
    assert not res["allclose"], kind


# ---- the reference's known-answer inputs ------------------------------------

def test_reference_warp_softmax_tile():
    """16x16 tile from srand(1234), uniform[-2,2] (fused/src/test_warp_softmax.cu:151-154):
    the C tile softmax equals a numpy softmax; rows sum to 1 when normalised."""
    x = c_oracle.rand_stream(1234, 256, 4.0).reshape(16, 16)
    assert x.min() >= -2.0 and x.max() <= 2.0
    for scale, norm in ((0.25, True), (1.0, True), (0.125, False)):
        out, mx, sm = c_oracle.tile_softmax(x, scale, norm)
        xs = x.astype(np.float64) * scale
        e = np.exp(xs - xs.max(1, keepdims=True))
        np.testing.assert_allclose(mx, xs.max(1), atol=1e-15)
        np.testing.assert_allclose(sm, e.sum(1), rtol=1e-14)
        np.testing.assert_allclose(out, e / e.sum(1, keepdims=True) if norm else e, rtol=1e-13)


def test_rand_stream_is_glibc_rand():
    import ctypes

    libc = ctypes.CDLL("libc.so.6")
    libc.srand(42)
    first = [libc.rand() for _ in range(3)]
    s = c_oracle.rand_stream(42, 3, 0.5)
    expect = (np.array(first, dtype=np.float32) / np.float32(2147483647) - np.float32(0.5)) * np.float32(0.5)
    np.testing.assert_array_equal(s, expect)


# ---- correctness metric (reference correctness.py:8-37) ----------------------

def test_check_correctness_semantics():
    r = np.array([1.0, -2.0, 0.0, 100.0], dtype=np.float32)
    o = np.array([1.011, -2.0, 0.005, 101.0], dtype=np.float32)
    res = ref.check_correctness(o, r, atol=1e-2, rtol=1e-2)
    assert res["allclose"]  # 0.011 <= 0.01 + 0.01; 0.005 <= 0.01; 1 <= 0.01 + 1
    assert abs(res["max_abs_err"] - 1.0) < 1e-6
    assert abs(res["max_rel_err"] - 0.005 / 1e-8) / (0.005 / 1e-8) < 1e-3
    o2 = o.copy()
    o2[0] = 1.03
    assert not ref.check_correctness(o2, r, atol=1e-2, rtol=1e-2)["allclose"]
    o3 = o.copy()
    o3[1] = np.nan
    assert not ref.check_correctness(o3, r)["allclose"]


def test_flops_formula():
    # C4: B=1 Hq=32 N=8192 d=128 causal
    assert ref.flops(1, 32, 8192, 128, causal=True) == 549755813888
    assert ref.flops(4, 12, 1024, 64) == 12884901888


# ---- separate query / key lengths (no reference counterpart: the reference
# binding rejects Nq != Nk).  Pinned against the square-causal oracle above
# and against torch's CPU scaled_dot_product_attention. -----------------------

def test_causal_mask_alignments():
    assert np.array_equal(ref.causal_mask(5, 5, True), np.triu(np.ones((5, 5), bool), 1))
    assert np.array_equal(ref.causal_mask(5, 5, 2), ref.causal_mask(5, 5, 1))
    assert ref.causal_mask(3, 7, False) is None
    tl = ref.causal_mask(2, 4, 1)
    br = ref.causal_mask(2, 4, 2)
    assert tl.tolist() == [[False, True, True, True], [False, False, True, True]]
    assert br.tolist() == [[False, False, False, True], [False, False, False, False]]
    # a row block of the full mask
    assert np.array_equal(ref.causal_mask(9, 12, 2, row0=3, rows=4),
                          ref.causal_mask(9, 12, 2)[3:7])


def test_top_left_with_longer_keys_equals_truncated_keys():
    q = rnd((1, 4, 24, 64), 31)
    k = rnd((1, 2, 70, 64), 32)
    v = rnd((1, 2, 70, 64), 33)
    got = ref.attention_reference(q, k, v, causal=1, return_f32=True)
    want = ref.attention_reference(q, k[:, :, :24], v[:, :, :24], causal=True, return_f32=True)
    np.testing.assert_allclose(got, want, atol=1e-6)


def test_bottom_right_is_tail_of_square_causal():
    n_k, n_q = 90, 13
    qf = rnd((2, 2, n_k, 128), 34)
    k = rnd((2, 1, n_k, 128), 35)
    v = rnd((2, 1, n_k, 128), 36)
    full = ref.attention_reference(qf, k, v, causal=True, return_f32=True)
    got = ref.attention_reference(qf[:, :, n_k - n_q:], k, v, causal=2, return_f32=True)
    np.testing.assert_allclose(got, full[:, :, n_k - n_q:], atol=1e-6)
    lse_full = ref.attention_lse(qf, k, causal=True)
    lse = ref.attention_lse(qf[:, :, n_k - n_q:], k, causal=2)
    np.testing.assert_allclose(lse, lse_full[:, :, n_k - n_q:], atol=1e-12)


def test_non_causal_rows_are_independent_of_query_count():
    q = rnd((1, 2, 50, 64), 37)
    k = rnd((1, 2, 20, 64), 38)
    v = rnd((1, 2, 20, 64), 39)
    whole = ref.attention_reference(q, k, v, return_f32=True)
    one = ref.attention_reference(q[:, :, 7:8], k, v, return_f32=True)
    np.testing.assert_allclose(one, whole[:, :, 7:8], atol=1e-6)
    # against the square oracle: the first 20 query rows with 20 keys
    sq = ref.attention_reference(q[:, :, :20], k, v, return_f32=True)
    np.testing.assert_allclose(whole[:, :, :20], sq, atol=1e-6)


@pytest.mark.parametrize("n_q,n_k,causal", [(1, 40, False), (7, 40, False), (7, 40, True),
                                            (40, 7, True), (40, 7, False)])
def test_matches_torch_sdpa_cpu(n_q, n_k, causal):
    import torch
    q = rnd((2, 4, n_q, 64), 40)
    k = rnd((2, 2, n_k, 64), 41)
    v = rnd((2, 2, n_k, 64), 42)
    got = ref.attention_reference(q, k, v, causal=causal, return_f32=True)
    ke, ve = ref.expand_kv_for_gqa(q, k, v)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).float(), torch.from_numpy(ke).float(),
        torch.from_numpy(ve).float(), is_causal=causal).numpy()
    np.testing.assert_allclose(got, want, atol=2e-6)
    np.testing.assert_allclose(ref.attention_f64(q, k, v, causal=causal), got, atol=2e-5)
    chunk = ref.attention_reference_chunked(q, k, v, causal=causal, rows=3, return_f32=True)
    np.testing.assert_allclose(chunk, got, atol=1e-6)


def test_rows_without_visible_keys_are_zero():
    # bottom-right with more queries than keys: query i sees keys j <= i - 30
    q = rnd((1, 1, 40, 64), 43)
    k = rnd((1, 1, 10, 64), 44)
    v = rnd((1, 1, 10, 64), 45)
    o = ref.attention_reference(q, k, v, causal=2, return_f32=True)
    assert np.all(o[:, :, :30] == 0)
    lse = ref.attention_lse(q, k, causal=2)
    assert np.all(np.isneginf(lse[:, :, :30])) and np.all(np.isfinite(lse[:, :, 30:]))
    # row 30 sees key 0 only
    np.testing.assert_allclose(o[0, 0, 30], v[0, 0, 0].astype(np.float32), atol=0)
    np.testing.assert_allclose(ref.attention_f64(q, k, v, causal=2)[0, 0, :30], 0)


# ---- explicit boolean attn_mask (no reference counterpart; torch SDPA's
# semantics, pinned against torch's CPU implementation) -----------------------

@pytest.mark.parametrize("mshape", [(2, 4, 9, 30), (2, 1, 9, 30), (9, 30), (2, 1, 1, 30)])
def test_bool_mask_matches_torch_sdpa_cpu(mshape):
    import torch
    q = rnd((2, 4, 9, 64), 50)
    k = rnd((2, 2, 30, 64), 51)
    v = rnd((2, 2, 30, 64), 52)
    r = np.random.default_rng(53)
    mask = r.random(mshape) < 0.7
    mask[..., 0] = True  # every row sees a key: torch gives NaN for empty rows
    got = ref.attention_reference(q, k, v, attn_mask=mask, return_f32=True)
    ke, ve = ref.expand_kv_for_gqa(q, k, v)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).float(), torch.from_numpy(ke).float(), torch.from_numpy(ve).float(),
        attn_mask=torch.from_numpy(np.ascontiguousarray(mask))).numpy()
    np.testing.assert_allclose(got, want, atol=2e-6)
    np.testing.assert_allclose(ref.attention_f64(q, k, v, attn_mask=mask), got, atol=2e-5)
    chunk = ref.attention_reference_chunked(q, k, v, attn_mask=mask, rows=4, return_f32=True)
    np.testing.assert_allclose(chunk, got, atol=1e-6)
    # LSE: closed form over the visible keys only
    lse = ref.attention_lse(q, k, attn_mask=mask)
    full = np.broadcast_to(mask, (2, 4, 9, 30))
    S = np.einsum("bhqd,bhkd->bhqk", q.astype(np.float64), ke.astype(np.float64)) / 8.0
    want_lse = np.log(np.where(full, np.exp(S), 0).sum(-1))
    np.testing.assert_allclose(lse, want_lse, atol=1e-10)


def test_bool_mask_special_cases():
    q = rnd((1, 2, 12, 64), 54)
    k = rnd((1, 2, 12, 64), 55)
    v = rnd((1, 2, 12, 64), 56)
    plain = ref.attention_reference(q, k, v, return_f32=True)
    ones = np.ones((12, 12), bool)
    np.testing.assert_array_equal(ref.attention_reference(q, k, v, attn_mask=ones, return_f32=True),
                                  plain)
    tril = np.tril(ones)
    np.testing.assert_allclose(ref.attention_reference(q, k, v, attn_mask=tril, return_f32=True),
                               ref.attention_reference(q, k, v, causal=True, return_f32=True),
                               atol=0)
    # a row with no visible key gives 0 (the kernels' 1/l -> 0 rule), not NaN
    m = ones.copy()
    m[3] = False
    o = ref.attention_reference(q, k, v, attn_mask=m, return_f32=True)
    assert np.all(o[:, :, 3] == 0) and np.all(np.isfinite(o))
    assert np.all(np.isneginf(ref.attention_lse(q, k, attn_mask=m)[:, :, 3]))
    # mask combined with causal: AND of the two
    r = np.random.default_rng(57).random((12, 12)) < 0.5
    np.testing.assert_allclose(
        ref.attention_reference(q, k, v, causal=True, attn_mask=r | np.eye(12, dtype=bool),
                                return_f32=True),
        ref.attention_reference(q, k, v, attn_mask=(r | np.eye(12, dtype=bool)) & tril,
                                return_f32=True), atol=0)


@pytest.mark.parametrize("n_q,n_k,mshape", [(9, 30, (2, 1, 1, 30)), (30, 30, (30, 30)),
                                            (13, 7, (2, 4, 13, 7))])
def test_bool_mask_with_is_causal_matches_torch_sdpa_cpu(n_q, n_k, mshape):
    """torch's CPU SDPA given both attn_mask and is_causal=True lets key j
    reach query i iff the mask allows it and j <= i (top-left): the oracle's
    causal=1 with the same mask."""
    import torch
    q = rnd((2, 4, n_q, 64), 58)
    k = rnd((2, 2, n_k, 64), 59)
    v = rnd((2, 2, n_k, 64), 60)
    mask = np.random.default_rng(61).random(mshape) < 0.7
    mask[..., 0] = True  # key 0 is visible to every row under top-left causal
    got = ref.attention_reference(q, k, v, causal=1, attn_mask=mask, return_f32=True)
    ke, ve = ref.expand_kv_for_gqa(q, k, v)
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q).float(), torch.from_numpy(ke).float(), torch.from_numpy(ve).float(),
        attn_mask=torch.from_numpy(np.ascontiguousarray(mask)), is_causal=True).numpy()
    np.testing.assert_allclose(got, want, atol=2e-6)
