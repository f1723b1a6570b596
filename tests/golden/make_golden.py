"""Writes the golden fixtures under tests/golden/ (run in the build container).

The reference ships no data fixtures, so the fixtures are produced by this
repository's oracle:
  * inputs: seeded CPU torch.Generator normal draws rounded to fp16, or the
    reference harnesses' own glibc rand() streams
    (fused/src/flash_mha_v2.cu:34-36,608-613: srand(42), uniform[-0.25,0.25],
    Q/K/V drawn interleaved; fused/src/test_warp_softmax.cu:151-154:
    srand(1234), uniform[-2,2], one 16x16 tile);
  * expected values: the fp32 numpy restatement of the reference math
    (oracle/attention_ref.py, fp16 output as the reference returns) and the
    long-double C oracle (output and LSE, stored as float32).

Usage:  python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
REPO = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, REPO)

from oracle import attention_ref as ref  # noqa: E402
from oracle import c_oracle  # noqa: E402

# (name, B, Hq, Hkv, N, D, causal, seed, std)
CASES = [
    ("c1_full_b1h1n512d64", 1, 1, 1, 512, 64, False, 0, 1.0),
    ("n1_d64", 1, 1, 1, 1, 64, False, 11, 1.0),
    ("n16_causal_d64", 1, 1, 1, 16, 64, True, 12, 1.0),
    ("n17_causal_d128", 1, 2, 2, 17, 128, True, 13, 1.0),
    ("n33_full_d128", 1, 2, 2, 33, 128, False, 14, 1.0),
    ("n127_causal_d64_b2", 2, 2, 2, 127, 64, True, 15, 1.0),
    ("gqa4_n200_causal_d128", 1, 4, 1, 200, 128, True, 16, 1.0),
    ("gqa4_n130_full_d64", 1, 4, 1, 130, 64, False, 17, 1.0),
    ("h8_n128_causal_d64", 1, 8, 8, 128, 64, True, 18, 1.0),
]


def torch_inputs(B, Hq, Hkv, N, D, seed, std):
    import torch

    g = torch.Generator("cpu").manual_seed(seed)
    q = (torch.randn(B, Hq, N, D, generator=g) * std).half().numpy()
    k = (torch.randn(B, Hkv, N, D, generator=g) * std).half().numpy()
    v = (torch.randn(B, Hkv, N, D, generator=g) * std).half().numpy()
    return q, k, v


def write_case(name, q, k, v, causal, scale):
    o16 = ref.attention_reference(q, k, v, causal=causal, scale=scale)
    o64, lse64 = c_oracle.attention_ld(q, k, v, causal=causal, scale=scale)
    np.savez_compressed(
        os.path.join(HERE, name + ".npz"),
        q=q, k=k, v=v, causal=np.array(causal), scale=np.array(scale, dtype=np.float64),
        out_f16=o16, out_exact=o64.astype(np.float32), lse_exact=lse64.astype(np.float32),
    )
    print(f"wrote {name}: q{q.shape} k{k.shape} causal={causal}")


def main():
    for name, B, Hq, Hkv, N, D, causal, seed, std in CASES:
        q, k, v = torch_inputs(B, Hq, Hkv, N, D, seed, std)
        write_case(name, q, k, v, causal, 1.0 / np.sqrt(D))

    # Reference V2 harness stream: srand(42), Q[i],K[i],V[i] interleaved.
    B, H, N, D = 1, 2, 64, 64
    total = B * H * N * D
    s = c_oracle.rand_stream(42, 3 * total, 0.5)
    q = s[0::3].astype(np.float16).reshape(B, H, N, D)
    k = s[1::3].astype(np.float16).reshape(B, H, N, D)
    v = s[2::3].astype(np.float16).reshape(B, H, N, D)
    for causal in (False, True):
        write_case(f"refv2_srand42_{'causal' if causal else 'full'}", q, k, v, causal,
                   1.0 / np.sqrt(D))

    # Reference warp-softmax known-answer tile: srand(1234), uniform[-2, 2].
    x = c_oracle.rand_stream(1234, 256, 4.0).reshape(16, 16)
    outs = {}
    for tag, scale, norm in (("s025_norm", 0.25, 1), ("s1_norm", 1.0, 1), ("s0125_unnorm", 0.125, 0)):
        o, m, sm = c_oracle.tile_softmax(x, scale, norm)
        outs[f"out_{tag}"] = o
        outs[f"max_{tag}"] = m
        outs[f"sum_{tag}"] = sm
    np.savez_compressed(os.path.join(HERE, "warp_softmax_srand1234.npz"), x=x, **outs)
    print("wrote warp_softmax_srand1234")


if __name__ == "__main__":
    main()
