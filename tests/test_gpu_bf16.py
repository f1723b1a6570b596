"""bfloat16 inputs on the GPU (flash_attention_forward_ex, the C ABI's dtype,
the SDPA patch).

No reference counterpart (the reference is binary16 only, and so are its
op names here: they still reject bfloat16).  The kernels are the binary16
ones with bfloat16 MFMAs and the probabilities rounded to bfloat16 before the
P V product.  Bar, against the numpy oracle in fp32 on the same (exactly
upcast) inputs: |O - O_ref| <= 4e-3 + 1.6e-2 |O_ref|.  bfloat16 keeps 8
significant bits, so the output rounding alone is up to 2^-8 |O| and each
probability carries up to 2^-8 relative rounding: this is the binary16 bar
(2e-3 + 1e-2 |O_ref|) widened for those 3 fewer bits; 1.6e-2 is torch's own
bfloat16 rtol.  It is an empirical bar for these inputs: where a peaked row's
largest weights cancel in V the error can exceed it while staying inside the
first-order rounding bound 2^-8 (sum_j P_j |V_j| + 2 |O_ref|), which
test_gpu_random_sweep.py checks.  LSE: the row sums add the bfloat16-rounded probabilities,
each within a relative 2^-8 of its exact value, so |LSE - LSE_ref| <=
log(1 + 2^-8) = 3.9e-3 (reached on rows whose softmax one key dominates).
"""
import numpy as np
import pytest
import torch

import flash_attn_sm75_cuda as _C
from flash_attention_sm75 import flash_attention_forward_ex
from flash_attention_sm75 import sdpa_patch as sp
from oracle import attention_ref as ref

pytestmark = pytest.mark.gpu

ATOL, RTOL = 4e-3, 1.6e-2
LSE_TOL = float(np.log1p(2.0 ** -8)) + 1e-5  # rounding bound, plus fp32 sums


def seeded(shape, seed):
    g = torch.Generator("cpu").manual_seed(seed)
    return torch.randn(*shape, generator=g).bfloat16()


def npf(t):
    return t.float().cpu().numpy()


def assert_parity(out, expect, label):
    res = ref.check_correctness(npf(out), expect, name=label, atol=ATOL, rtol=RTOL)
    print(f"  {label}: max_abs={res['max_abs_err']:.3e}", flush=True)
    assert res["allclose"], res


CASES = [
    # B, Hq, Hkv, Nq, Nk, D, causal
    (1, 8, 2, 200, 200, 128, True),
    (2, 4, 4, 129, 129, 64, False),
    (1, 4, 1, 1000, 1000, 128, True),
    (2, 8, 8, 64, 64, 64, True),
    (3, 32, 8, 1, 3000, 128, False),        # decode (split-K path)
    (2, 14, 2, 1, 777, 64, True),           # decode, Qwen2-0.5B heads
    (1, 8, 2, 7, 300, 128, "bottom_right"),
    (1, 2, 2, 300, 77, 64, "bottom_right"),  # rows that see no key
]


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", CASES)
def test_bf16_matches_oracle(device, B, Hq, Hkv, Nq, Nk, D, causal):
    print(f"[bf16] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal}", flush=True)
    q, k, v = seeded((B, Hq, Nq, D), 1), seeded((B, Hkv, Nk, D), 2), seeded((B, Hkv, Nk, D), 3)
    o, lse = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                        causal=causal, return_lse=True)
    torch.cuda.synchronize()
    assert o.dtype == torch.bfloat16
    code = {False: 0, True: 1, "bottom_right": 2}[causal]
    expect = ref.attention_reference(npf(q), npf(k), npf(v), causal=code, return_f32=True)
    assert_parity(o, expect, f"Nq{Nq} Nk{Nk} D{D}")
    lse_ref = ref.attention_lse(npf(q), npf(k), causal=code)
    got = lse.cpu().numpy()
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(got), fin)
    np.testing.assert_allclose(got[fin], lse_ref[fin], atol=LSE_TOL, rtol=0)


@pytest.mark.parametrize("B,Hq,Hkv,Nq,Nk,D,causal", [
    (3, 7, 1, 340, 535, 64, False),
    (2, 8, 1, 418, 1697, 128, False),
    (3, 28, 4, 79, 141, 64, True),
    (1, 4, 1, 3, 900, 128, False),          # decode rows
])
def test_bf16_peaked_rows(device, B, Hq, Hkv, Nq, Nk, D, causal):
    """Scale 0.3 (2.4x-3.4x the default): most rows are dominated by one key,
    where the bfloat16 rounding of that probability sets the LSE error."""
    print(f"[bf16 peaked] B={B} Hq={Hq} Hkv={Hkv} Nq={Nq} Nk={Nk} D={D} causal={causal}", flush=True)
    q, k, v = seeded((B, Hq, Nq, D), 11), seeded((B, Hkv, Nk, D), 12), seeded((B, Hkv, Nk, D), 13)
    o, lse = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device), causal=causal,
                                        scale=0.3, return_lse=True)
    torch.cuda.synchronize()
    code = {False: 0, True: 1}[causal]
    expect = ref.attention_reference(npf(q), npf(k), npf(v), causal=code, scale=0.3,
                                     return_f32=True)
    assert_parity(o, expect, f"peaked Nq{Nq} Nk{Nk} D{D}")
    lse_ref = ref.attention_lse(npf(q), npf(k), causal=code, scale=0.3)
    got = lse.cpu().numpy()
    err = float(np.abs(got - lse_ref).max())
    print(f"  LSE max_abs={err:.3e} (bound {LSE_TOL:.3e})", flush=True)
    np.testing.assert_allclose(got, lse_ref, atol=LSE_TOL, rtol=0)


@pytest.mark.parametrize("D", [64, 128])
def test_bf16_kernels_agree(device, D):
    """Every prefill kernel shape and schedule in bfloat16 (forced by the
    policy switch) against the oracle on sampled heads; the static and
    dynamic schedules and the 256-row workgroups bitwise against the
    128-row ones."""
    B, Hq, Hkv, N = 2, 32, 8, 1100
    q, k, v = seeded((B, Hq, N, D), 4), seeded((B, Hkv, N, D), 5), seeded((B, Hkv, N, D), 6)
    qd, kd, vd = q.to(device), k.to(device), v.to(device)
    outs = {}
    try:
        for pol in (0, 1, 2, 3, 4, 5):  # auto, 128-row, 256-row, dynamic, key split, pairs
            _C.set_kernel_policy(pol)
            outs[pol] = flash_attention_forward_ex(qd, kd, vd, causal=True)
    finally:
        _C.set_kernel_policy(0)
    torch.cuda.synchronize()
    assert torch.equal(outs[1], outs[3])
    assert torch.equal(outs[1], outs[2])
    group = Hq // Hkv
    for h in (0, 17, 31):
        exp = ref.attention_reference(npf(q[:, h:h + 1]), npf(k[:, h // group:h // group + 1]),
                                      npf(v[:, h // group:h // group + 1]), causal=True,
                                      return_f32=True)
        for pol, o in outs.items():
            assert_parity(o[:, h:h + 1], exp, f"policy {pol} head {h}")


def test_bf16_boolean_mask(device):
    B, Hq, Hkv, N, D = 2, 4, 2, 300, 64
    q, k, v = seeded((B, Hq, N, D), 7), seeded((B, Hkv, N, D), 8), seeded((B, Hkv, N, D), 9)
    g = torch.Generator("cpu").manual_seed(10)
    mask = torch.rand(B, 1, N, N, generator=g) < 0.7
    mask[..., 0] = True  # every row sees a key
    o = flash_attention_forward_ex(q.to(device), k.to(device), v.to(device),
                                   attn_mask=mask.to(device))
    torch.cuda.synchronize()
    expect = ref.attention_reference(npf(q), npf(k), npf(v), return_f32=True,
                                     attn_mask=mask.numpy())
    assert_parity(o, expect, "masked")


def test_reference_ops_stay_fp16(device):
    """The reference-named ops keep the reference's FP16-only contract."""
    x = seeded((1, 2, 64, 64), 11).to(device)
    with pytest.raises(RuntimeError, match="must be FP16"):
        _C.flash_attention_forward(x, x, x, False, 0.125)
    with pytest.raises(RuntimeError, match="same dtype"):
        flash_attention_forward_ex(x, x.half(), x)


def test_bf16_qwen2_prefill_and_decode(device):
    """A random-init Qwen2 in bfloat16 (the dtype HF models now default to):
    with the patch every attention call (prefill and KV-cache decode) runs on
    the kernel; last-token logits stay close to torch's SDPA in bfloat16 and
    agree on every clear top-1."""
    transformers = pytest.importorskip("transformers")
    cfg = transformers.Qwen2Config(
        vocab_size=2000, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
        num_attention_heads=4, num_key_value_heads=1, max_position_embeddings=4096,
        attn_implementation="sdpa")
    torch.manual_seed(0)
    model = transformers.Qwen2ForCausalLM(cfg).to(torch.bfloat16).to("cuda").eval()
    g = torch.Generator("cpu").manual_seed(12)
    ids = torch.randint(0, 2000, (2, 260), generator=g).to(device)
    prompt, steps = ids[:, :250], ids[:, 250:]

    def run():
        with torch.no_grad():
            out = model(input_ids=prompt, use_cache=True)
            logits = [out.logits[:, -1]]
            cache = out.past_key_values
            for t in range(steps.size(1)):
                out = model(input_ids=steps[:, t:t + 1], past_key_values=cache, use_cache=True)
                cache = out.past_key_values
                logits.append(out.logits[:, -1])
        return torch.stack(logits, 1).float()

    plain = run()
    sp.apply_patch()
    sp.reset_stats()
    try:
        pat = run()
        stats = sp.patch_stats()
    finally:
        sp.remove_patch()
    torch.cuda.synchronize()
    print(f"  stats: {stats}", flush=True)
    assert stats["fallback"] == 0
    assert stats["flash"] == 2 * (1 + steps.size(1))
    diff = (plain - pat).abs().max().item()
    scale = plain.abs().max().item()
    print(f"  max |dlogit| = {diff:.3e} (max |logit| {scale:.3e})", flush=True)
    assert diff <= 2e-2 + 5e-2 * scale
    top2 = plain.topk(2, dim=-1)
    decided = (top2.values[..., 0] - top2.values[..., 1]) > 2 * diff
    assert torch.equal(plain.argmax(-1)[decided], pat.argmax(-1)[decided])
