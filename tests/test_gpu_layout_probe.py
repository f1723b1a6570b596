"""Device probes of the hardware semantics the attention kernels rely on
(needs a GPU): the v_mfma_f32_32x32x16 operand and accumulator layouts, the
ds_read_b64_tr_b16 transposing read, and the half-wave exchange of
v_permlane32_swap.  The kernels' own parity tests cover these end to end;
these pin each one on its own, so a wrong assumption names itself.

The probes live in tests/probe/layout_probe.hip (built by
__graft_entry__.build() into tests/probe/liblayout_probe.so) and use the
product's own device helpers (fa_kernel_common.h).
"""
import ctypes
import os

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

HERE = os.path.dirname(os.path.abspath(__file__))
PROBE = os.path.join(HERE, "probe", "liblayout_probe.so")


@pytest.fixture(scope="module")
def probe():
    if not os.path.exists(PROBE):
        pytest.fail(f"{PROBE} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(PROBE)
    for f in ("fa_probe_mfma", "fa_probe_tr16", "fa_probe_halves"):
        getattr(lib, f).restype = ctypes.c_int
    lib.fa_probe_mfma.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int]
    lib.fa_probe_tr16.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int, ctypes.c_void_p]
    lib.fa_probe_halves.argtypes = [ctypes.c_void_p] * 3
    return lib


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mfma_32x32x16_layout(device, probe, dtype):
    """Each lane loads A, B in the claimed operand layouts and stores C in the
    claimed accumulator layout: the stored matrix is A @ B exactly (small
    integers) only if all three layouts hold."""
    print(f"[probe] mfma 32x32x16 {dtype}", flush=True)
    g = torch.Generator("cpu").manual_seed(5)
    a = torch.randint(-4, 5, (32, 16), generator=g).to(dtype)
    b = torch.randint(-4, 5, (16, 32), generator=g).to(dtype)
    c = torch.full((32, 32), float("nan"), dtype=torch.float32, device=device)
    ad, bd = a.to(device), b.to(device)
    rc = probe.fa_probe_mfma(ad.data_ptr(), bd.data_ptr(), c.data_ptr(),
                             int(dtype == torch.bfloat16))
    assert rc == 0
    want = a.float().numpy() @ b.float().numpy()
    np.testing.assert_array_equal(c.cpu().numpy(), want)


def test_transposing_read_mapping(device, probe):
    """ds_read_b64_tr_b16: within each 16-lane group, lane i's element j is
    the 16-bit word at (address of group lane 4j + i/4) + i % 4."""
    print("[probe] ds_read_b64_tr_b16", flush=True)
    n = 4096
    mem = torch.arange(n, dtype=torch.int32).to(torch.int16)  # word w holds w
    rng = np.random.default_rng(7)
    addr = torch.from_numpy(rng.integers(0, n // 4, 64).astype(np.int32) * 4)
    out = torch.zeros(64, 4, dtype=torch.int16, device=device)
    memd, addrd = mem.to(device), addr.to(device)
    assert probe.fa_probe_tr16(addrd.data_ptr(), memd.data_ptr(), n, out.data_ptr()) == 0
    got = out.cpu().numpy().astype(np.int64) & 0xFFFF
    a = addr.numpy()
    want = np.empty((64, 4), dtype=np.int64)
    for lane in range(64):
        grp, i = divmod(lane, 16)
        for j in range(4):
            want[lane, j] = a[16 * grp + 4 * j + i // 4] + i % 4
    np.testing.assert_array_equal(got, want)


def test_half_wave_exchange(device, probe):
    """halves_max / halves_sum combine lanes l and l ^ 32 (the two halves of
    a query's keys in the S^T accumulator)."""
    print("[probe] v_permlane32_swap", flush=True)
    x = torch.randn(64, generator=torch.Generator("cpu").manual_seed(9))
    xd = x.to(device)
    mx = torch.empty(64, device=device)
    sm = torch.empty(64, device=device)
    assert probe.fa_probe_halves(xd.data_ptr(), mx.data_ptr(), sm.data_ptr()) == 0
    xn = x.numpy()
    partner = xn[np.arange(64) ^ 32]
    np.testing.assert_array_equal(mx.cpu().numpy(), np.maximum(xn, partner))
    np.testing.assert_allclose(sm.cpu().numpy(), xn + partner, rtol=0, atol=0)
