"""Prints the gfx950 unit rates that bound the fused attention step (MFMA,
VALU, LDS, launch gap), from tests/probe/libhw_rates.so (hw_rates.hip).

    python tests/probe/hw_rates.py

Measurement infrastructure, not a test: nothing in the product imports it.
Each figure is the fastest of three runs.
"""
import ctypes
import os
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libhw_rates.so")


def load():
    lib = ctypes.CDLL(LIB)
    for f, args in (("fa_rate_mix", [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
                    ("fa_rate_valu", [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
                    ("fa_rate_lds", [ctypes.c_int, ctypes.c_int, ctypes.c_int]),
                    ("fa_rate_launch", [ctypes.c_longlong, ctypes.c_int])):
        getattr(lib, f).argtypes = args
        getattr(lib, f).restype = ctypes.c_double
    return lib


def best(f, *args, low=True):
    vals = [f(*args) for _ in range(3)]
    if any(v < 0 for v in vals):
        raise RuntimeError(f"probe failed: {vals}")
    return min(vals) if low else max(vals)


def main():
    lib = load()
    rows = []
    mfma = {w: best(lib.fa_rate_mix, 0, w, 2000) for w in (1, 2)}
    for w in (1, 2):
        rows.append((f"16 MFMA 32x32x16 f16, {w} wave(s)/SIMD", f"{mfma[w]:.1f} ns per wave-iteration",
                     f"{mfma[w] / 16:.2f} ns per MFMA"))
    names = ("v_fma_f32", "v_exp_f32", "v_max3_f32", "v_cvt_pk_f16_f32 / v_dot2c_f32_f16")
    for op, name in enumerate(names):
        r = best(lib.fa_rate_valu, op, 4, 4000)
        rows.append((f"{name}, 4 waves/SIMD", f"{r:.2f} ns per wave-instruction", ""))
    for nv in (64, 112):
        for w in (1, 2):
            r = best(lib.fa_rate_mix, nv, w, 2000)
            rows.append((f"16 MFMA + {nv} VALU interleaved, {w} wave(s)/SIMD",
                         f"{r:.1f} ns per wave-iteration",
                         f"MFMA alone {mfma[w]:.1f}"))
    for op, name in ((0, "ds_read_b128"), (1, "ds_read_b64_tr_b16")):
        r = best(lib.fa_rate_lds, op, 4, 4000, low=False)
        rows.append((f"{name}, 4 waves/SIMD", f"{r:.0f} bytes/ns per CU", ""))
    for clocks in (10000, 20000):
        r = best(lib.fa_rate_launch, clocks, 100)
        rows.append((f"back-to-back launches, spin {clocks} clocks", f"{r:.2f} us per launch", ""))
    w0 = max(len(r[0]) for r in rows)
    for a, b, c in rows:
        print(f"{a:<{w0}}  {b:<34} {c}", flush=True)


if __name__ == "__main__":
    sys.exit(main())
