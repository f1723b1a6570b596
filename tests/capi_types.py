"""ctypes mirror of include/flash_attn_sm75.h used by the C-ABI tests."""
import ctypes
import os

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB = os.path.join(REPO, "flash-attention-sm75-register-fused_amd", "src",
                   "libflash_attn_sm75_hip.so")


class Params(ctypes.Structure):
    _fields_ = [(n, t) for n, t in [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("batch", ctypes.c_int64), ("heads_q", ctypes.c_int64), ("heads_kv", ctypes.c_int64),
        ("seq_len", ctypes.c_int64), ("head_dim", ctypes.c_int64),
        ("q_stride_b", ctypes.c_int64), ("q_stride_h", ctypes.c_int64), ("q_stride_n", ctypes.c_int64),
        ("k_stride_b", ctypes.c_int64), ("k_stride_h", ctypes.c_int64), ("k_stride_n", ctypes.c_int64),
        ("v_stride_b", ctypes.c_int64), ("v_stride_h", ctypes.c_int64), ("v_stride_n", ctypes.c_int64),
        ("o_stride_b", ctypes.c_int64), ("o_stride_h", ctypes.c_int64), ("o_stride_n", ctypes.c_int64),
        ("scale", ctypes.c_float), ("causal", ctypes.c_int), ("stream", ctypes.c_void_p),
        ("seq_len_kv", ctypes.c_int64),
        ("workspace", ctypes.c_void_p), ("workspace_bytes", ctypes.c_int64),
        ("mask_bits", ctypes.c_void_p), ("mask_stride_b", ctypes.c_int64),
        ("mask_stride_h", ctypes.c_int64), ("mask_stride_q", ctypes.c_int64),
        ("dtype", ctypes.c_int),
        ("mask_keys", ctypes.c_void_p), ("mask_keys_stride_b", ctypes.c_int64),
        ("mask_keys_stride_k", ctypes.c_int64),
        ("mask_ranges", ctypes.c_void_p), ("mask_ranges_stride_b", ctypes.c_int64),
        ("mask_ranges_stride_h", ctypes.c_int64), ("mask_ranges_stride_q", ctypes.c_int64),
    ]]


FA_CAUSAL_NONE, FA_CAUSAL_TOP_LEFT, FA_CAUSAL_BOTTOM_RIGHT = 0, 1, 2
FA_DTYPE_FP16, FA_DTYPE_BF16 = 0, 1


def _strides(*names):
    return [(f"{n}_stride_{d}", ctypes.c_int64) for n in names for d in ("b", "h", "n")]


class BwdParams(ctypes.Structure):
    """fa_bwd_params."""
    _fields_ = [
        ("q", ctypes.c_void_p), ("k", ctypes.c_void_p), ("v", ctypes.c_void_p),
        ("o", ctypes.c_void_p), ("dout", ctypes.c_void_p), ("lse", ctypes.c_void_p),
        ("dq", ctypes.c_void_p), ("dk", ctypes.c_void_p), ("dv", ctypes.c_void_p),
        ("batch", ctypes.c_int64), ("heads_q", ctypes.c_int64), ("heads_kv", ctypes.c_int64),
        ("seq_len", ctypes.c_int64), ("seq_len_kv", ctypes.c_int64), ("head_dim", ctypes.c_int64),
    ] + _strides("q", "k", "v", "o", "do", "dq", "dk", "dv") + [
        ("scale", ctypes.c_float), ("causal", ctypes.c_int), ("dtype", ctypes.c_int),
        ("stream", ctypes.c_void_p), ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_int64),
        ("mask_bits", ctypes.c_void_p), ("mask_stride_b", ctypes.c_int64),
        ("mask_stride_h", ctypes.c_int64), ("mask_stride_q", ctypes.c_int64),
        ("mask_ranges", ctypes.c_void_p), ("mask_ranges_stride_b", ctypes.c_int64),
        ("mask_ranges_stride_h", ctypes.c_int64), ("mask_ranges_stride_q", ctypes.c_int64),
    ]
