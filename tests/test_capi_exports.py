"""The C-ABI library loads and exports every function include/*.h declares.

Calls made here never reach the device: they exercise argument validation,
which runs before the first HIP call.
"""
import ctypes
import glob
import os
import re

import pytest

from capi_types import LIB, REPO, Params


def declared_functions():
    names = []
    for hdr in glob.glob(os.path.join(REPO, "include", "*.h")):
        text = open(hdr).read()
        text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
        for m in re.finditer(r"\b([a-z_][a-z0-9_]*)\s*\(", text):
            name = m.group(1)
            prefix = text[:m.start()].rstrip()
            if name in {"sizeof", "if", "return"}:
                continue
            # a declaration: preceded by a type, ends with ');'
            tail = text[m.end():text.find(";", m.end()) + 1]
            if tail.endswith(");") and re.search(r"(void|int|int64_t|char\s*\*|char)\s*\**$", prefix):
                names.append(name)
    return sorted(set(names))


@pytest.fixture(scope="module")
def lib():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built: run __graft_entry__.build()")
    lib = ctypes.CDLL(LIB)
    lib.fa_sm75_forward.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_forward.restype = ctypes.c_int
    lib.fa_sm75_naive_forward.argtypes = [ctypes.POINTER(Params), ctypes.c_void_p]
    lib.fa_sm75_naive_forward.restype = ctypes.c_int
    lib.fa_sm75_last_error.restype = ctypes.c_char_p
    lib.fa_sm75_status_string.restype = ctypes.c_char_p
    lib.fa_sm75_set_contiguous_strides.argtypes = [ctypes.POINTER(Params)]
    return lib


def test_header_declares_expected_entry_points():
    names = declared_functions()
    for n in ("fa_sm75_forward", "fa_sm75_naive_forward", "fa_sm75_last_error",
              "fa_sm75_status_string", "fa_sm75_abi_version", "fa_sm75_set_contiguous_strides",
              "fa_sm75_workspace_size", "fa_sm75_forward_noalloc", "fa_sm75_pack_mask",
              "fa_sm75_backward",
              "fa_sm75_backward_workspace_size", "fa_sm75_set_contiguous_bwd_strides",
              "launch_flash_attention_forward", "launch_flash_attention_forward_scalar",
              "launch_flash_attention_forward_wmma_qk", "launch_naive_attention"):
        assert n in names, n


def test_every_declared_symbol_is_exported(lib):
    for name in declared_functions():
        assert hasattr(lib, name), f"{name} declared in include/ but not exported"


def make(lib, **kw):
    p = Params()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = 1, 4, 2, 64, 128
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    p.q = p.k = p.v = p.o = 0x10000
    p.scale = 0.125
    for k, v in kw.items():
        setattr(p, k, v)
    return p


def test_contiguous_strides(lib):
    p = make(lib)
    assert (p.q_stride_n, p.q_stride_h, p.q_stride_b) == (128, 64 * 128, 4 * 64 * 128)
    assert (p.k_stride_n, p.k_stride_h, p.k_stride_b) == (128, 64 * 128, 2 * 64 * 128)


def test_contiguous_strides_separate_kv_length(lib):
    p = Params()
    p.batch, p.heads_q, p.heads_kv, p.seq_len, p.head_dim = 2, 4, 2, 5, 64
    p.seq_len_kv = 300
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    assert (p.q_stride_n, p.q_stride_h, p.q_stride_b) == (64, 5 * 64, 4 * 5 * 64)
    assert (p.o_stride_n, p.o_stride_h, p.o_stride_b) == (64, 5 * 64, 4 * 5 * 64)
    assert (p.k_stride_n, p.k_stride_h, p.k_stride_b) == (64, 300 * 64, 2 * 300 * 64)
    assert (p.v_stride_n, p.v_stride_h, p.v_stride_b) == (64, 300 * 64, 2 * 300 * 64)


@pytest.mark.parametrize("kw,status,msg", [
    (dict(head_dim=96), 2, b"supports head_dim=64 or 128, got 96"),
    (dict(heads_kv=3), 3, b"not divisible"),
    (dict(heads_kv=0), 3, b"heads_kv must be positive"),
    (dict(seq_len=-1), 1, b"non-negative"),
    (dict(q=0), 1, b"must not be NULL"),
    (dict(k=0x10008), 4, b"16-byte aligned"),
    (dict(q_stride_n=100), 4, b"multiples of 8"),
    (dict(scale=float("inf")), 1, b"finite"),
    (dict(causal=3), 1, b"causal must be 0, 1 (top-left) or 2 (bottom-right)"),
    (dict(causal=-1), 1, b"causal must be"),
    (dict(seq_len_kv=-5), 1, b"non-negative"),
    (dict(seq_len_kv=1 << 30), 5, b"exceeds the supported maximum"),
    (dict(workspace=0x10004, workspace_bytes=64), 4, b"workspace must be 16-byte aligned"),
    (dict(workspace_bytes=-1), 1, b"workspace_bytes must be non-negative"),
    (dict(dtype=2), 1, b"dtype must be 0 (binary16) or 1 (bfloat16)"),
    (dict(dtype=-1), 1, b"dtype must be"),
])
def test_validation_errors(lib, kw, status, msg):
    p = make(lib, **kw)
    assert lib.fa_sm75_forward(ctypes.byref(p)) == status
    assert msg in lib.fa_sm75_last_error()
    assert lib.fa_sm75_status_string(status) != b"unknown status"


def test_noalloc_validation(lib):
    """fa_sm75_forward_noalloc validates like fa_sm75_forward and rejects a
    caller workspace, all before touching the device."""
    lib.fa_sm75_forward_noalloc.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_forward_noalloc.restype = ctypes.c_int
    assert lib.fa_sm75_forward_noalloc(None) == 1
    p = make(lib, head_dim=96)
    assert lib.fa_sm75_forward_noalloc(ctypes.byref(p)) == 2
    assert b"supports head_dim=64 or 128, got 96" in lib.fa_sm75_last_error()
    p = make(lib, workspace=0x10000, workspace_bytes=4096)
    assert lib.fa_sm75_forward_noalloc(ctypes.byref(p)) == 1
    assert b"takes no workspace" in lib.fa_sm75_last_error()
    p = make(lib, workspace_bytes=16)
    assert lib.fa_sm75_forward_noalloc(ctypes.byref(p)) == 1
    assert lib.fa_sm75_forward_noalloc(ctypes.byref(make(lib, seq_len=0))) == 0


def test_null_params(lib):
    assert lib.fa_sm75_forward(None) == 1


def test_empty_problem_is_a_noop(lib):
    for kw in (dict(batch=0), dict(seq_len=0), dict(heads_q=0)):
        p = make(lib, q=0, k=0, v=0, o=0, **kw)
        assert lib.fa_sm75_forward(ctypes.byref(p)) == 0


def test_naive_validation(lib):
    p = make(lib, head_dim=96)
    p2 = make(lib, head_dim=100)
    assert lib.fa_sm75_naive_forward(ctypes.byref(p), None) == 1  # workspace NULL
    assert lib.fa_sm75_naive_forward(ctypes.byref(p2), None) == 2  # not a multiple of 8
    p3 = make(lib, seq_len_kv=65)
    assert lib.fa_sm75_naive_forward(ctypes.byref(p3), ctypes.c_void_p(0x10000)) == 1
    assert b"seq_len_kv == seq_len" in lib.fa_sm75_last_error()
    p4 = make(lib, dtype=1)
    assert lib.fa_sm75_naive_forward(ctypes.byref(p4), ctypes.c_void_p(0x10000)) == 1
    assert b"binary16 only" in lib.fa_sm75_last_error()


def test_workspace_size(lib):
    lib.fa_sm75_workspace_size.argtypes = [ctypes.POINTER(Params)]
    lib.fa_sm75_workspace_size.restype = ctypes.c_int64
    # prefill: 8 queue counters, 256 bytes apart, when the 128-row kernel's
    # dynamic schedule runs -- under AUTO for long launches only (at least
    # 1024 key-tile steps per resident workgroup; 512 workgroups without a
    # device), always under DYNAMIC, never under NARROW or WIDE
    p = make(lib)
    assert lib.fa_sm75_workspace_size(ctypes.byref(p)) == 0
    long_call = make(lib, batch=2, heads_q=64, heads_kv=8, seq_len=16384, causal=1)
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(long_call))
    assert lib.fa_sm75_workspace_size(ctypes.byref(long_call)) == 8 * 256
    short_call = make(lib, batch=1, heads_q=32, heads_kv=8, seq_len=8192, causal=1)
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(short_call))
    assert lib.fa_sm75_workspace_size(ctypes.byref(short_call)) == 0
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    try:
        for policy, want in ((1, 0), (2, 0), (3, 8 * 256), (4, 0), (5, 0)):
            lib.fa_sm75_set_kernel_policy(policy)
            assert lib.fa_sm75_workspace_size(ctypes.byref(p)) == want, policy
            assert lib.fa_sm75_workspace_size(ctypes.byref(long_call)) == want, policy
    finally:
        lib.fa_sm75_set_kernel_policy(0)
    # decode: 4 query heads over 2 KV heads, one query row, 8192 keys
    p = make(lib, seq_len=1, seq_len_kv=8192)
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    ws = lib.fa_sm75_workspace_size(ctypes.byref(p))
    rows, units, d = 2, 2, 128
    assert ws > 0 and ws % (units * rows * (d + 2) * 4) == 0
    # invalid parameters: 0, and the last error is left alone
    lib.fa_sm75_forward(ctypes.byref(make(lib, head_dim=96)))
    msg = lib.fa_sm75_last_error()
    assert lib.fa_sm75_workspace_size(ctypes.byref(make(lib, head_dim=48, seq_len=1))) == 0
    assert lib.fa_sm75_last_error() == msg
    # a forced kernel policy never takes the split-K path
    try:
        lib.fa_sm75_set_kernel_policy(1)
        assert lib.fa_sm75_workspace_size(ctypes.byref(p)) == 0
        lib.fa_sm75_set_kernel_policy(3)
        assert lib.fa_sm75_workspace_size(ctypes.byref(p)) == 8 * 256
    finally:
        lib.fa_sm75_set_kernel_policy(0)


def test_pack_mask_validation(lib):
    f = lib.fa_sm75_pack_mask
    f.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p, ctypes.c_void_p]
    f.restype = ctypes.c_int
    assert f(0x1000, 1, 1, 1, 0, 0, 0, 0, 1, 0x1000, None) == 0      # empty: no-op
    assert f(0x1000, -1, 1, 1, 8, 0, 0, 0, 1, 0x1000, None) == 1
    assert b"non-negative" in lib.fa_sm75_last_error()
    assert f(0x1000, 1, 1, 1, 8, 0, 0, -1, 1, 0x1000, None) == 1
    assert f(0, 1, 1, 1, 8, 0, 0, 0, 1, 0x1000, None) == 1
    assert f(0x1000, 1, 1, 1, 8, 0, 0, 0, 1, 0x1004, None) == 4
    assert b"8-byte aligned" in lib.fa_sm75_last_error()


def test_mask_param_validation(lib):
    p = make(lib, mask_bits=0x1004)
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 4
    p = make(lib, mask_bits=0x1000, mask_stride_q=-1)
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 1
    p = make(lib, mask_bits=0x1000, mask_stride_q=1, seq_len_kv=200)  # 200 keys need 4 words
    lib.fa_sm75_set_contiguous_strides(ctypes.byref(p))
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 1
    assert b"below ceil(seq_len_kv / 64)" in lib.fa_sm75_last_error()
    p = make(lib, mask_bits=0x1000)
    assert lib.fa_sm75_naive_forward(ctypes.byref(p), ctypes.c_void_p(0x1000)) == 1
    assert b"naive path takes no mask" in lib.fa_sm75_last_error()


def test_mask_keys_validation(lib):
    """Key-padding bytes: exclusive with mask_bits, non-negative strides, not
    on the naive path (all rejected before any device work)."""
    p = make(lib, mask_keys=0x1000, mask_bits=0x1000)
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 1
    assert b"exclusive" in lib.fa_sm75_last_error()
    for field in ("mask_keys_stride_b", "mask_keys_stride_k"):
        p = make(lib, mask_keys=0x1001, **{field: -1})
        assert lib.fa_sm75_forward(ctypes.byref(p)) == 1
        assert b"mask_keys strides" in lib.fa_sm75_last_error()
    p = make(lib, mask_keys=0x1001)
    assert lib.fa_sm75_naive_forward(ctypes.byref(p), ctypes.c_void_p(0x1000)) == 1
    assert b"naive path takes no mask" in lib.fa_sm75_last_error()


def test_mask_ranges_validation(lib):
    """Row spans of visible keys: only with mask_bits, 8-byte aligned,
    non-negative strides; the packing entry that writes them needs the
    output (all rejected before any device work)."""
    p = make(lib, mask_ranges=0x2000)
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 1
    assert b"needs mask_bits" in lib.fa_sm75_last_error()
    p = make(lib, mask_bits=0x1000, mask_ranges=0x2004)
    assert lib.fa_sm75_forward(ctypes.byref(p)) == 4
    assert b"8-byte aligned" in lib.fa_sm75_last_error()
    for field in ("mask_ranges_stride_b", "mask_ranges_stride_h", "mask_ranges_stride_q"):
        p = make(lib, mask_bits=0x1000, mask_ranges=0x2000, **{field: -1})
        assert lib.fa_sm75_forward(ctypes.byref(p)) == 1
        assert b"mask_ranges strides" in lib.fa_sm75_last_error()
    f = lib.fa_sm75_pack_mask_ranges
    f.argtypes = [ctypes.c_void_p] + [ctypes.c_int64] * 8 + [ctypes.c_void_p] * 3
    f.restype = ctypes.c_int
    assert f(0x1000, 1, 1, 1, 8, 0, 0, 0, 1, 0x1000, None, None) == 1
    assert b"ranges must not be NULL" in lib.fa_sm75_last_error()
    assert f(0x1000, 1, 1, 1, 8, 0, 0, 0, 1, 0x1000, 0x2004, None) == 4
    assert f(0x1000, 1, 1, 1, 1 << 31, 0, 0, 0, 1, 0x1000, 0x2000, None) == 5


def test_abi_version(lib):
    assert lib.fa_sm75_abi_version() == 7


def test_kernel_policy_switch(lib):
    lib.fa_sm75_set_kernel_policy.argtypes = [ctypes.c_int]
    assert lib.fa_sm75_get_kernel_policy() == 0
    assert lib.fa_sm75_set_kernel_policy(6) == 1
    assert lib.fa_sm75_set_kernel_policy(-1) == 1
    try:
        for p in (1, 2, 3, 4, 5, 0):
            assert lib.fa_sm75_set_kernel_policy(p) == 0
            assert lib.fa_sm75_get_kernel_policy() == p
    finally:
        lib.fa_sm75_set_kernel_policy(0)
