"""Parity of the gfx950 fused forward against the CPU oracle (needs a GPU).

Bar (north star): |O - O_ref| <= 2e-3 + 1e-2 * |O_ref| elementwise
(torch.allclose semantics of reference src/reference/correctness.py:24 with
atol=2e-3, rtol=1e-2), against the reference math path restated in numpy
(fp32, the reference's op order) and against the long-double closed form.
Against the unrounded fp32 oracle (and the long-double closed form) the
max-abs error is also asserted, max |O - O_ref| <= 2e-3 (the north star's
max-abs bar, reference src/reference/correctness.py:13-14 computes it).  It
is not asserted against the oracle's own fp16-rounded output: fp16 values
in [2, 4) have an ulp of 1.95e-3, so two correctly rounded results can
differ by about one ulp there.

Inputs are drawn from a CPU torch.Generator and copied to the device, so the
same seed gives the same data on every machine.
"""
import math
import os

import numpy as np
import pytest
import torch

import flash_attn_sm75_cuda as _C
from flash_attention_sm75 import flash_attention_forward, flash_attention_forward_lse
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-3, 1e-2
HERE = os.path.dirname(os.path.abspath(__file__))


def make_inputs(B, Hq, Hkv, N, D, seed=0, std=1.0):
    g = torch.Generator("cpu").manual_seed(seed)
    q = (torch.randn(B, Hq, N, D, generator=g) * std).half()
    k = (torch.randn(B, Hkv, N, D, generator=g) * std).half()
    v = (torch.randn(B, Hkv, N, D, generator=g) * std).half()
    return q, k, v


def assert_parity(out, expect, label, max_abs=ATOL):
    """allclose(atol=2e-3, rtol=1e-2) and, unless ``max_abs`` is None (a
    comparison with an fp16-rounded expectation), max-abs <= ``max_abs``."""
    out = out.detach().float().cpu().numpy() if torch.is_tensor(out) else out
    res = ref.check_correctness(out, expect, name=label, atol=ATOL, rtol=RTOL)
    print(f"  {label}: max_abs={res['max_abs_err']:.3e} mean_abs={res['mean_abs_err']:.3e}",
          flush=True)
    assert res["allclose"], res
    if max_abs is not None:
        assert res["max_abs_err"] <= max_abs, res
    return res


def run_case(B, Hq, Hkv, N, D, causal, seed=0, std=1.0, scale=None):
    print(f"[case] B={B} Hq={Hq} Hkv={Hkv} N={N} D={D} causal={causal} seed={seed}", flush=True)
    q, k, v = make_inputs(B, Hq, Hkv, N, D, seed, std)
    dev = torch.device("cuda", 0)
    out = flash_attention_forward(q.to(dev), k.to(dev), v.to(dev), causal=causal, scale=scale)
    torch.cuda.synchronize()
    expect = ref.attention_reference_chunked(q.numpy(), k.numpy(), v.numpy(), causal=causal,
                                             scale=scale, return_f32=True)
    assert out.shape == q.shape and out.dtype == torch.float16
    return assert_parity(out, expect, f"B{B} H{Hq}/{Hkv} N{N} D{D} c{int(causal)}")


# ---- the committed golden fixtures ----------------------------------------

GOLDEN = sorted(
    f for f in os.listdir(os.path.join(HERE, "golden"))
    if f.endswith(".npz") and not f.startswith("warp_softmax")
)


@pytest.mark.parametrize("name", GOLDEN)
def test_golden_fixture(device, name):
    z = np.load(os.path.join(HERE, "golden", name))
    print(f"[golden] {name} q{z['q'].shape}", flush=True)
    q, k, v = (torch.from_numpy(z[x]).to(device) for x in ("q", "k", "v"))
    causal, scale = bool(z["causal"]), float(z["scale"])
    out, lse = flash_attention_forward_lse(q, k, v, causal=causal, scale=scale)
    torch.cuda.synchronize()
    assert_parity(out, z["out_exact"], name + " vs closed form")
    assert_parity(out, z["out_f16"].astype(np.float32), name + " vs reference math (fp16)",
                  max_abs=None)
    np.testing.assert_allclose(lse.cpu().numpy(), z["lse_exact"], atol=2e-4, rtol=1e-5)


# ---- the reference's own test shapes ---------------------------------------

# reference tests/test_flash_d128.py:42-63, tests/test_flash_forward.py:43-53,
# tests/test_flash_wmma_qk.py:41-52 (B, H, N, D, causal)
REFERENCE_CASES = sorted(set([
    (1, 8, 128, 64, False), (1, 8, 512, 64, False), (1, 8, 1024, 64, True),
    (1, 8, 128, 128, False), (1, 8, 256, 128, False), (1, 8, 512, 128, False),
    (1, 8, 1024, 128, False), (2, 8, 256, 128, False), (1, 16, 512, 128, False),
    (1, 8, 128, 128, True), (1, 8, 256, 128, True), (1, 8, 512, 128, True),
    (1, 8, 1024, 128, True),
    (1, 8, 256, 64, False), (1, 16, 128, 64, False), (2, 8, 128, 64, False),
    (1, 8, 128, 64, True), (1, 8, 256, 64, True), (2, 8, 256, 64, False),
    (1, 8, 512, 64, True),
    # reference tests/test_correctness.py:69-76 edge cases
    (1, 1, 1, 64, False), (1, 1, 16, 64, True), (1, 32, 128, 64, True),
]))


@pytest.mark.parametrize("B,H,N,D,causal", REFERENCE_CASES)
def test_reference_shapes(device, B, H, N, D, causal):
    run_case(B, H, H, N, D, causal, seed=42)


# ---- sequence tails, GQA groupings ----------------------------------------

@pytest.mark.parametrize("N", [2, 15, 31, 63, 64, 65, 127, 129, 200, 255, 257, 1000])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_sequence_tails(device, N, D, causal):
    run_case(1, 2, 2, N, D, causal, seed=N)


@pytest.mark.parametrize("Hq,Hkv", [(8, 2), (8, 1), (32, 8), (12, 4)])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("D", [64, 128])
def test_gqa(device, Hq, Hkv, causal, D):
    run_case(2, Hq, Hkv, 300, D, causal, seed=Hq * 10 + Hkv)


# ---- BASELINE configurations ------------------------------------------------

def test_c1_full(device):
    run_case(1, 1, 1, 512, 64, False, seed=0)


def test_c2_full_with_lse(device):
    print("[case] C2 B=4 H=12 N=1024 D=64 full + LSE", flush=True)
    q, k, v = make_inputs(4, 12, 12, 1024, 64, seed=1)
    out, lse = flash_attention_forward_lse(q.to(device), k.to(device), v.to(device), causal=False)
    torch.cuda.synchronize()
    expect = ref.attention_reference_chunked(q.numpy(), k.numpy(), v.numpy(), return_f32=True)
    assert_parity(out, expect, "C2")
    lse_ref = ref.attention_lse(q.numpy(), k.numpy(), causal=False)
    np.testing.assert_allclose(lse.cpu().numpy(), lse_ref, atol=2e-4, rtol=1e-5)


def test_c3_causal(device):
    run_case(4, 8, 8, 2048, 64, True, seed=2)


def heads_per_unit(B, Hq, Hkv, per_unit=1, shift=0):
    """(batch, query head) pairs, ``per_unit`` query heads of each (batch, KV
    head) unit at different positions of its group (position (u + shift*b) %
    group, then spread by group / per_unit).  The kernels give each unit its
    own XCD share (static order) or queue (dynamic schedule), so one head per
    unit already covers every XCD and every queue of a full-size launch."""
    group = Hq // Hkv
    out = []
    for b in range(B):
        for u in range(Hkv):
            first = (u + shift * b) % group
            for i in range(per_unit):
                out.append((b, u * group + (first + i * (group // per_unit)) % group))
    return out


def _oracle_slices(q, k, v, pairs, causal):
    """Unrounded fp32 oracle (the reference's op order with torch on the
    host CPU, all threads) for (batch, query head) pairs, all rows; a causal
    row block evaluates only the keys up to its diagonal (the others are
    hidden from every row of the block)."""
    out = []
    for b, h in pairs:
        out.append(ref.attention_reference_torch_cpu(
            q[b:b + 1], k[b:b + 1], v[b:b + 1], causal=causal, rows=2048, heads=[h],
            return_f32=True, skip_hidden=True)[0, 0].numpy())
    return out


def _check_units(q, k, v, out, causal, pairs, label):
    got = out.float().cpu()
    worst = 0.0
    for (b, h), expect in zip(pairs, _oracle_slices(q, k, v, pairs, causal)):
        res = assert_parity(got[b, h].numpy(), expect, f"{label} b{b} h{h}")
        worst = max(worst, res["max_abs_err"])
    print(f"  {label}: {len(pairs)} (batch, head) slices, worst max_abs={worst:.3e}", flush=True)


def test_heads_per_unit_layout():
    """The C5 sample holds two distinct heads of every unit, each inside its
    unit's group; C4's full sample is every head once."""
    pairs = heads_per_unit(2, 64, 8, per_unit=2, shift=3)
    assert len(set(pairs)) == 32
    for b in range(2):
        for u in range(8):
            hs = {h for bb, h in pairs if bb == b and h // 8 == u}
            assert len(hs) == 2
    assert sorted(h for _, h in heads_per_unit(1, 32, 8, per_unit=4)) == list(range(32))


def test_c4_causal_gqa_full_size(device):
    """C4 at full size: every one of the 32 query heads, every row, against
    the unrounded fp32 oracle (allclose 2e-3 / 1e-2 and max-abs <= 2e-3)."""
    print("[case] C4 B=1 Hq=32 Hkv=8 N=8192 D=128 causal", flush=True)
    q, k, v = make_inputs(1, 32, 8, 8192, 128, seed=3)
    out = flash_attention_forward(q.to(device), k.to(device), v.to(device), causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item()
    # causal row 0 attends only to key 0: O[0] == V[kv head][0] exactly
    assert torch.equal(out[0, :, 0].cpu(), v[0].repeat_interleave(4, 0)[:, 0])
    _check_units(q, k, v, out, True, heads_per_unit(1, 32, 8, per_unit=4), "C4")


def test_c5_long_context_stress(device):
    """C5: N(0, 0.5^2) inputs, K x4 on a random 5% of rows (softmax max
    rescaling stress), B=2 Hq=64 Hkv=8 N=16384 D=128 causal.  Two query heads
    of each of the 16 (batch, KV head) units, at different positions of the
    unit's group (32 of the 128 slices), every row, against the unrounded fp32
    oracle: each unit is one queue of the dynamic schedule this launch runs."""
    print("[case] C5 B=2 Hq=64 Hkv=8 N=16384 D=128 causal, K x4 on 5% rows", flush=True)
    g = torch.Generator("cpu").manual_seed(4)
    B, Hq, Hkv, N, D = 2, 64, 8, 16384, 128
    q = (torch.randn(B, Hq, N, D, generator=g) * 0.5).half()
    k = torch.randn(B, Hkv, N, D, generator=g) * 0.5
    v = (torch.randn(B, Hkv, N, D, generator=g) * 0.5).half()
    rows = torch.rand(B, Hkv, N, generator=g) < 0.05
    k = torch.where(rows[..., None], k * 4, k).half()
    out = flash_attention_forward(q.to(device), k.to(device), v.to(device), causal=True)
    torch.cuda.synchronize()
    assert torch.isfinite(out).all().item()
    assert torch.equal(out[:, :, 0].cpu(), v.repeat_interleave(8, 1)[:, :, 0])
    _check_units(q, k, v, out, True, heads_per_unit(B, Hq, Hkv, per_unit=2, shift=3), "C5")


def test_warp_softmax_known_answer(device):
    """The reference's in-register softmax known-answer test (reference
    flash-attention-sm75-fused/src/test_warp_softmax.cu:151-213: a 16x16
    tile of (rand()/RAND_MAX - 0.5) * 4 after srand(1234), row softmax at
    scales 0.25 and 1 (normalised) and 0.125 (row max and sum)) run through
    the fused kernel: Q's rows are one-hot (Q[i, i] = 1), K[j, i] = x[i][j]
    rounded to fp16, V's rows one-hot (V[j, j] = 1), so S = scale * x and
    O[i, :16] is the tile's row softmax, and LSE_i = max_i + ln(sum_i).

    Expected values: the long-double softmax of the fp16-rounded tile.  O is
    held to the parity bar (its entries are fp16).  The reference holds its
    fp32 row max and sum to 1e-4; the kernel exposes them only as
    LSE = max + ln(sum), whose sum adds the fp16-rounded probabilities (the
    values the P V product takes).  So LSE is held to 1e-4 against that
    statement (sum of fp16(exp(s x - max))), and to ln(1 + 2^-11) = 4.9e-4,
    the relative error of one fp16 rounding, against the exact softmax."""
    from oracle import c_oracle

    z = np.load(os.path.join(HERE, "golden", "warp_softmax_srand1234.npz"))
    x16 = z["x"].astype(np.float16)
    tile = x16.astype(np.float32)
    q = torch.zeros(1, 1, 16, 64, dtype=torch.float16)
    k = torch.zeros(1, 1, 16, 64, dtype=torch.float16)
    v = torch.zeros(1, 1, 16, 64, dtype=torch.float16)
    idx = torch.arange(16)
    q[0, 0, idx, idx] = 1
    v[0, 0, idx, idx] = 1
    k[0, 0, :, :16] = torch.from_numpy(x16).T
    lse_bar = math.log1p(2.0 ** -11)
    for scale, norm in ((0.25, 1), (1.0, 1), (0.125, 0)):
        print(f"[kat] warp softmax scale={scale} normalised={norm}", flush=True)
        out, lse = flash_attention_forward_lse(q.to(device), k.to(device), v.to(device),
                                               causal=False, scale=scale)
        torch.cuda.synchronize()
        want, mx, sm = c_oracle.tile_softmax(tile, scale, True)
        got = out[0, 0].float().cpu().numpy()
        assert np.all(got[:, 16:] == 0)
        assert_parity(got[:, :16], want.astype(np.float32), f"kat scale {scale}")
        err = np.abs(lse[0, 0].cpu().numpy().astype(np.float64) - (mx + np.log(sm)))
        print(f"  kat scale {scale}: LSE max err {err.max():.3e} (bar {lse_bar:.3e})", flush=True)
        assert err.max() <= lse_bar
        p16 = np.exp(scale * tile.astype(np.float64) - mx[:, None]).astype(np.float16)
        lse_rounded_p = mx + np.log(p16.astype(np.float64).sum(axis=1))
        err_p = np.abs(lse[0, 0].cpu().numpy().astype(np.float64) - lse_rounded_p)
        print(f"  kat scale {scale}: LSE vs rounded-P sum {err_p.max():.3e} (bar 1e-4)", flush=True)
        assert err_p.max() <= 1e-4
        if not norm:  # the unnormalised variant: exp(s x - max) = O * exp(LSE - max)
            want_u, _, _ = c_oracle.tile_softmax(tile, scale, False)
            got_u = got[:, :16] * np.exp(lse[0, 0].cpu().numpy().astype(np.float64) - mx)[:, None]
            assert_parity(got_u.astype(np.float32), want_u.astype(np.float32),
                          f"kat scale {scale} unnormalised")


# ---- scale, strides, streams, determinism ---------------------------------

@pytest.mark.parametrize("scale", [0.0, -0.125, 1.0, 0.01])
def test_scales(device, scale):
    run_case(1, 2, 2, 190, 64, True, seed=7, scale=scale)
    run_case(1, 2, 1, 130, 128, False, seed=8, scale=scale)


def test_noncontiguous_inputs(device):
    q, k, v = make_inputs(2, 4, 2, 100, 64, seed=9)
    qt = q.transpose(1, 2).contiguous().to(device).transpose(1, 2)  # [B,H,N,D] view
    assert not qt.is_contiguous()
    a = flash_attention_forward(qt, k.to(device), v.to(device), causal=True)
    b = flash_attention_forward(q.to(device), k.to(device), v.to(device), causal=True)
    assert torch.equal(a, b)


def test_side_stream_and_determinism(device):
    q, k, v = (x.to(device) for x in make_inputs(1, 8, 2, 777, 128, seed=10))
    base = flash_attention_forward(q, k, v, causal=True)
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        other = flash_attention_forward(q, k, v, causal=True)
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    assert torch.equal(base, other)


def test_output_is_fresh_and_inputs_untouched(device):
    q, k, v = (x.to(device) for x in make_inputs(1, 2, 2, 64, 64, seed=11))
    q0, k0, v0 = q.clone(), k.clone(), v.clone()
    out = flash_attention_forward(q, k, v)
    torch.cuda.synchronize()
    assert out.data_ptr() not in (q.data_ptr(), k.data_ptr(), v.data_ptr())
    assert torch.equal(q, q0) and torch.equal(k, k0) and torch.equal(v, v0)


# ---- compatibility ops (reference pytorch_extension.cpp:124-129) ----------

@pytest.mark.parametrize("op", ["flash_attention_forward_scalar", "flash_attention_forward_wmma_qk"])
def test_d64_compat_ops(device, op):
    q, k, v = (x.to(device) for x in make_inputs(1, 4, 4, 300, 64, seed=12))
    out = getattr(_C, op)(q, k, v, True, 0.125)
    main = _C.flash_attention_forward(q, k, v, True, 0.125)
    torch.cuda.synchronize()
    assert torch.equal(out, main)
    with pytest.raises(RuntimeError, match="supports head_dim=64 only"):
        q2 = torch.zeros(1, 1, 16, 128, dtype=torch.float16, device=device)
        getattr(_C, op)(q2, q2, q2, False, 0.1)


@pytest.mark.parametrize("N,D,causal", [(1, 64, False), (16, 64, True), (300, 128, True),
                                        (1024, 64, False), (129, 96, True)])
def test_naive_op(device, N, D, causal):
    print(f"[naive] N={N} D={D} causal={causal}", flush=True)
    q, k, v = make_inputs(2, 3, 3, N, D, seed=13)
    scale = 1.0 / math.sqrt(D)
    out = _C.naive_attention_forward(q.to(device), k.to(device), v.to(device), causal, scale)
    torch.cuda.synchronize()
    expect = ref.attention_reference(q.numpy(), k.numpy(), v.numpy(), causal=causal,
                                     scale=scale, return_f32=True)
    assert_parity(out, expect, f"naive N{N} D{D}")


def test_binding_shape_errors(device):
    z = lambda *s: torch.zeros(*s, dtype=torch.float16, device=device)  # noqa: E731
    with pytest.raises(RuntimeError, match="heads mismatch"):
        _C.flash_attention_forward(z(1, 6, 16, 64), z(1, 4, 16, 64), z(1, 4, 16, 64), False, 1.0)
    with pytest.raises(RuntimeError, match="seq_len mismatch"):
        _C.flash_attention_forward(z(1, 4, 16, 64), z(1, 4, 8, 64), z(1, 4, 8, 64), False, 1.0)
    with pytest.raises(RuntimeError, match="must be FP16"):
        _C.flash_attention_forward(z(1, 4, 16, 64).float(), z(1, 4, 16, 64), z(1, 4, 16, 64), False, 1.0)
    with pytest.raises(RuntimeError, match="must be contiguous"):
        t = z(1, 16, 4, 64).transpose(1, 2)
        _C.flash_attention_forward(t, t, t, False, 1.0)
    with pytest.raises(RuntimeError, match="naive_attention: Q, K, V must have identical shapes"):
        _C.naive_attention_forward(z(1, 4, 16, 64), z(1, 2, 16, 64), z(1, 2, 16, 64), False, 1.0)


def test_backward_raises_after_forward(device):
    # reference tests/test_api.py:31-41
    q, k, v = (x.to(device) for x in make_inputs(1, 8, 8, 128, 64, seed=14))
    q.requires_grad_(True)
    out = flash_attention_forward(q, k, v)
    with pytest.raises(NotImplementedError, match="Backward pass is not implemented"):
        out.sum().backward()


def test_empty_sequence(device):
    q = torch.zeros(1, 2, 0, 64, dtype=torch.float16, device=device)
    out = flash_attention_forward(q, q, q, causal=True)
    assert out.shape == q.shape


def test_single_hip_runtime_loaded(device):
    """The library and torch share one HIP runtime in the process."""
    maps = open("/proc/self/maps").read().splitlines()
    libs = {line.split()[-1] for line in maps if "libamdhip64" in line}
    print("  libamdhip64 mapped:", sorted(libs), flush=True)
    assert len({os.path.realpath(p) for p in libs}) == 1, libs
