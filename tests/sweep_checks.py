"""Checks shared by the seeded parity sweeps (tests/test_gpu_random_sweep.py,
tests/test_gpu_mask_sweep.py): one case's forward (O, LSE) and, for small
sizes, its gradients, through the kernels against the numpy oracle.

Bars (those of the dedicated tests):
  * O: |O - O_ref| <= 2e-3 + 1e-2 |O_ref| (binary16, O_ref in fp32); for
    bfloat16 the first-order rounding bound 2^-8 (sum_j P_j |V_j| + 2 |O_ref|),
    O_ref and sum_j P_j |V_j| (the oracle's attention over |V|) in float64;
  * LSE: the same infinite entries (rows that see no key), finite ones within
    1e-3 + 1e-4 |LSE_ref| (binary16) or log(1 + 2^-8) (bfloat16), LSE_ref in
    float64;
  * gradients (Nq <= 400 and Nk <= 800): |G - R| <= a max|R| + r |R| with
    (a, r) = (2e-3, 1e-2) or (1e-2, 4e-2), R the float64 closed form with the
    row term rowsum(dO o O) taken from the kernel's own O.
"""
import numpy as np
import torch

from flash_attention_sm75 import flash_attention, flash_attention_forward_ex
from oracle import attention_ref as ref

CAUSAL = {0: False, 1: True, 2: "bottom_right"}


def check_case(device, q, k, v, mask, code, scale, bf16, g, strided=False):
    """q, k, v: CPU tensors (binary16 or bfloat16, any strides); mask: a CPU
    bool tensor broadcastable to [B, Hq, Nq, Nk], or None; code: causal mode
    (0 none, 1 top-left, 2 bottom-right), applied together with the mask; g:
    the CPU generator the case's dO is drawn from."""
    B, Hq, Nq, D = q.shape
    Hkv, Nk = k.shape[1], k.shape[2]
    dt = q.dtype
    npf = lambda t: t.float().cpu().numpy()
    m_np = None if mask is None else mask.numpy()
    md = None if mask is None else mask.to(device)
    qd, kd, vd = (t.to(device) for t in (q, k, v))  # .to keeps the strides
    if strided:  # a size-1 dimension's stride does not matter
        assert Nq == 1 or qd.stride(2) == Hq * D
        assert Nk == 1 or kd.stride(2) == Hkv * D
    o, lse = flash_attention_forward_ex(qd, kd, vd, causal=CAUSAL[code], scale=scale,
                                        return_lse=True, attn_mask=md)
    torch.cuda.synchronize()
    want = ref.attention_reference(npf(q), npf(k), npf(v), causal=code, scale=scale,
                                   return_f32=True, attn_mask=m_np)
    got = npf(o)
    assert np.isfinite(got).all()
    if bf16:
        want = ref.attention_f64(npf(q), npf(k), npf(v), causal=code, scale=scale, attn_mask=m_np)
        spv = ref.attention_f64(npf(q), npf(k), np.abs(npf(v)), causal=code, scale=scale,
                                attn_mask=m_np)
        bound = 2.0 ** -8 * (spv + 2 * np.abs(want)) * 1.01 + 2e-6
    else:
        bound = 2e-3 + 1e-2 * np.abs(want)
    err = np.abs(got - want)
    assert np.all(err <= bound), float((err / bound).max())
    lse_ref = ref.attention_lse(npf(q), npf(k), causal=code, scale=scale, attn_mask=m_np)
    gl = lse.cpu().numpy()
    fin = np.isfinite(lse_ref)
    assert np.array_equal(np.isfinite(gl), fin)
    if bf16:
        np.testing.assert_allclose(gl[fin], lse_ref[fin], atol=float(np.log1p(2.0 ** -8)) + 1e-5,
                                   rtol=0)
    else:
        np.testing.assert_allclose(gl[fin], lse_ref[fin], atol=1e-3, rtol=1e-4)
    if Nq > 400 or Nk > 800:
        return
    leaves = [t.detach().requires_grad_() for t in (qd, kd, vd)]
    do = torch.randn(B, Hq, Nq, D, generator=g).to(dt)
    out = flash_attention(*leaves, causal=CAUSAL[code], scale=scale, attn_mask=md)
    out.backward(do.to(device))
    torch.cuda.synchronize()
    wants = ref.attention_backward_f64(npf(q), npf(k), npf(v), npf(do), causal=code, scale=scale,
                                       attn_mask=m_np, delta_from_o=npf(out.detach()))
    ba, br = (1e-2, 4e-2) if bf16 else (2e-3, 1e-2)
    for name, leaf, w in zip(("dQ", "dK", "dV"), leaves, wants):
        gg = npf(leaf.grad).astype(np.float64)
        sc = max(float(np.abs(w).max()) if w.size else 0.0, 1e-2)
        worst = float((np.abs(gg - w) / (ba * sc + br * np.abs(w) + 1e-30)).max()) if w.size else 0.0
        print(f"  {name}: worst/bar={worst:.3f}", flush=True)
        assert np.isfinite(gg).all(), name
        assert worst <= 1.0, (name, worst)
