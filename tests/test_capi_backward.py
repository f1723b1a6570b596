"""C-ABI validation of fa_sm75_backward (no device needed: every check runs
before the first HIP call)."""
import ctypes
import os

import pytest

from capi_types import LIB, BwdParams


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_backward.argtypes = [ctypes.POINTER(BwdParams)]
    lib.fa_sm75_backward.restype = ctypes.c_int
    lib.fa_sm75_backward_workspace_size.argtypes = [ctypes.POINTER(BwdParams)]
    lib.fa_sm75_backward_workspace_size.restype = ctypes.c_int64
    lib.fa_sm75_set_contiguous_bwd_strides.argtypes = [ctypes.POINTER(BwdParams)]
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    return lib


def make(lib, **kw):
    p = BwdParams()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = 2, 8, 2, 100, 128
    for k, v in kw.items():
        if k in ("batch", "heads_q", "heads_kv", "seq_len", "seq_len_kv", "head_dim"):
            setattr(p, k, v)
    lib.fa_sm75_set_contiguous_bwd_strides(ctypes.byref(p))
    for name in ("q", "k", "v", "o", "dout", "lse", "dq", "dk", "dv", "workspace"):
        setattr(p, name, 0x10000)
    p.workspace_bytes = lib.fa_sm75_backward_workspace_size(ctypes.byref(p))
    p.scale = 0.088
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_contiguous_strides(lib):
    p = make(lib, seq_len_kv=300)
    assert (p.q_stride_n, p.q_stride_h, p.q_stride_b) == (128, 100 * 128, 8 * 100 * 128)
    assert (p.dq_stride_n, p.do_stride_h, p.o_stride_b) == (128, 100 * 128, 8 * 100 * 128)
    assert (p.k_stride_n, p.k_stride_h, p.k_stride_b) == (128, 300 * 128, 2 * 300 * 128)
    assert (p.dv_stride_n, p.dk_stride_h, p.dv_stride_b) == (128, 300 * 128, 2 * 300 * 128)


def test_workspace_size(lib):
    # 520 bytes per (batch, query head, 64 query rows): the stats record, then the tile's key span
    assert lib.fa_sm75_backward_workspace_size(ctypes.byref(make(lib))) == 2 * 8 * 2 * 520
    assert lib.fa_sm75_backward_workspace_size(ctypes.byref(make(lib, seq_len=64))) == 2 * 8 * 520
    assert lib.fa_sm75_backward_workspace_size(ctypes.byref(make(lib, seq_len=0))) == 0
    assert lib.fa_sm75_backward_workspace_size(None) == 0


@pytest.mark.parametrize("kw,status,msg", [
    (dict(head_dim=96), 2, b"supports head_dim=64 or 128"),
    (dict(heads_kv=3), 3, b"not divisible"),
    (dict(heads_kv=0), 3, b"heads_kv must be positive"),
    (dict(batch=-1), 1, b"non-negative"),
    (dict(scale=float("nan")), 1, b"scale must be finite"),
    (dict(causal=3), 1, b"causal must be 0, 1 (top-left) or 2 (bottom-right)"),
    (dict(dtype=2), 1, b"dtype must be 0 (binary16) or 1 (bfloat16)"),
    (dict(dq=0), 1, b"must not be NULL"),
    (dict(dout=0), 1, b"must not be NULL"),
    (dict(workspace=0), 1, b"must not be NULL"),
    (dict(lse=0), 1, b"lse must not be NULL"),
    (dict(lse=0x10002), 4, b"lse must be 4-byte aligned"),
    (dict(dk=0x10008), 4, b"16-byte aligned"),
    (dict(do_stride_n=132), 4, b"multiples of 8"),
    (dict(dq_stride_h=-8), 1, b"non-negative"),
    (dict(dv_stride_n=120), 1, b"row stride must be at least head_dim"),
    (dict(workspace_bytes=100), 1, b"below the required"),
    (dict(seq_len_kv=1 << 30), 5, b"exceeds the supported maximum"),
    (dict(q_stride_n=1 << 24), 5, b"exceeds 2^31 bytes"),
    (dict(mask_bits=0x10004), 4, b"mask_bits must be 8-byte aligned"),
    (dict(mask_bits=0x10000, mask_stride_h=-1), 1, b"mask strides must be non-negative"),
    (dict(mask_bits=0x10000, mask_stride_q=1), 1, b"mask row stride 1 is below"),
    (dict(mask_bits=0x10000, mask_stride_q=1 << 22), 5, b"mask row stride exceeds 2^31"),
])
def test_validation_errors(lib, kw, status, msg):
    p = make(lib, **kw)
    assert lib.fa_sm75_backward(ctypes.byref(p)) == status
    assert msg in lib.fa_sm75_last_error()


def test_null_params(lib):
    assert lib.fa_sm75_backward(None) == 1


def test_empty_problems_are_noops(lib):
    for kw in (dict(batch=0), dict(heads_q=0), dict(seq_len=0, seq_len_kv=0)):
        p = make(lib, **kw)
        for name in ("q", "k", "v", "o", "dout", "lse", "dq", "dk", "dv", "workspace"):
            setattr(p, name, 0)
        assert lib.fa_sm75_backward(ctypes.byref(p)) == 0, kw


def test_no_query_rows_needs_only_kv_pointers(lib):
    """seq_len == 0 with keys: dK = dV = 0 are still written, so K, V, dK and
    dV must be valid; Q-side pointers and the workspace may be NULL (the
    zero-size check passes, the launch is not reached without them)."""
    p = make(lib, seq_len=0, seq_len_kv=50)
    for name in ("q", "o", "dout", "lse", "dq", "workspace"):
        setattr(p, name, 0)
    p.dk = 0
    assert lib.fa_sm75_backward(ctypes.byref(p)) == 1
    assert b"must not be NULL" in lib.fa_sm75_last_error()
