"""In-tree build of the gfx950 library and its PyTorch binding.

Produces, next to the Python package in ``src/``:

* ``libflash_attn_sm75_hip.so`` -- the HIP kernels and the C ABI declared in
  ``include/flash_attn_sm75.h`` (hipcc, ``--offload-arch=gfx950``);
* ``flash_attn_sm75_cuda<EXT_SUFFIX>`` -- the pybind11 module with the
  reference's op names (g++ against libtorch; links the library above with an
  ``$ORIGIN`` rpath).

Run ``python build_native.py`` from anywhere; ``__graft_entry__.build()`` calls
:func:`build`.  Compilation happens every call (no staleness checks), which is
what the repository's build check expects.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
import sysconfig
import tempfile
from concurrent.futures import ThreadPoolExecutor

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
REPO_DIR = os.path.dirname(PKG_DIR)
CSRC = os.path.join(PKG_DIR, "csrc")
OUT_DIR = os.path.join(PKG_DIR, "src")
INCLUDE = os.path.join(REPO_DIR, "include")
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")

HIP_LIB_NAME = "libflash_attn_sm75_hip.so"
EXT_NAME = "flash_attn_sm75_cuda"

# The fused kernel's instances (fa_fwd_d*.hip) are separate translation units
# so that they compile in parallel.
HIP_SOURCES = [
    "fa_fwd_d128.hip", "fa_fwd_d128_mask.hip", "fa_fwd_d128_w8.hip", "fa_fwd_d128_mask_w8.hip",
    "fa_fwd_d128_ks.hip",
    "fa_fwd_d64.hip", "fa_fwd_d64_mask.hip", "fa_fwd_d64_w8.hip", "fa_fwd_d64_mask_w8.hip",
    "fa_fwd_d64_ks.hip",
    "fa_fwd_d128_bf16.hip", "fa_fwd_d128_mask_bf16.hip", "fa_fwd_d128_w8_bf16.hip",
    "fa_fwd_d128_mask_w8_bf16.hip", "fa_fwd_d128_ks_bf16.hip",
    "fa_fwd_d64_bf16.hip", "fa_fwd_d64_mask_bf16.hip", "fa_fwd_d64_w8_bf16.hip",
    "fa_fwd_d64_mask_w8_bf16.hip", "fa_fwd_d64_ks_bf16.hip",
    "fa_fwd_d128_keys.hip", "fa_fwd_d64_keys.hip", "fa_fwd_d128_keys_bf16.hip",
    "fa_fwd_d64_keys_bf16.hip",
    "fa_bwd_d128.hip", "fa_bwd_d64.hip", "fa_bwd_d128_mask.hip", "fa_bwd_d64_mask.hip",
    "fa_bwd.hip",
    "fa_fwd.hip", "fa_decode.hip", "fa_mask.hip", "fa_naive.hip", "fa_capi.hip",
]

# Packed-FP32 VALU forms are disabled for all device code.  The atomic
# optimizer is off: it would turn the fused kernel's single-lane ticket
# request into a wave-wide one whose result is waited for at once, where the
# kernel wants the request in flight during its last step.
HIPCC_FLAGS = [
    "--offload-arch=gfx950",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-mllvm", "-amdgpu-atomic-optimizer-strategy=None",
]


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print("+", " ".join(cmd), flush=True)
    res = subprocess.run(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True)
    out = "\n".join(
        line for line in res.stdout.splitlines()
        # hipcc's host pass does not know the device-only feature name.
        if "packed-fp32-ops" not in line
    )
    if res.returncode != 0:
        raise RuntimeError(f"build step failed ({res.returncode}): {' '.join(cmd)}\n{out}")
    if verbose and out.strip():
        print(out)


def hip_lib_path() -> str:
    return os.path.join(OUT_DIR, HIP_LIB_NAME)


def ext_path() -> str:
    return os.path.join(OUT_DIR, EXT_NAME + sysconfig.get_config_var("EXT_SUFFIX"))


def build_hip_lib(verbose: bool = False) -> str:
    """Compiles every HIP source to an object (in parallel, in a temporary
    directory) and links the shared library."""
    hipcc = os.path.join(ROCM, "bin", "hipcc")
    out = hip_lib_path()
    tmp = out + ".tmp"
    objdir = tempfile.mkdtemp(prefix="fa_sm75_build_")
    try:
        objs = [os.path.join(objdir, os.path.splitext(s)[0] + ".o") for s in HIP_SOURCES]
        cmds = [[hipcc, *HIPCC_FLAGS, f"-I{INCLUDE}", f"-I{CSRC}", "-c",
                 os.path.join(CSRC, s), "-o", o] for s, o in zip(HIP_SOURCES, objs)]
        jobs = max(1, min(len(cmds), int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        _run([hipcc, "--offload-arch=gfx950", "-shared", "-fPIC", *objs, "-o", tmp], verbose)
    finally:
        shutil.rmtree(objdir, ignore_errors=True)
    os.replace(tmp, out)
    return out


def build_binding(verbose: bool = False) -> str:
    import torch.utils.cpp_extension as ce

    out = ext_path()
    tmp = out + ".tmp"
    incs = ce.include_paths("cuda")
    libdirs = ce.library_paths("cuda")
    py_inc = sysconfig.get_paths()["include"]
    import torch

    abi = int(torch._C._GLIBCXX_USE_CXX11_ABI)
    cmd = [
        "g++", "-O2", "-std=c++17", "-fPIC", "-shared",
        "-D__HIP_PLATFORM_AMD__=1", "-DUSE_ROCM=1",
        f"-DTORCH_EXTENSION_NAME={EXT_NAME}", "-DTORCH_API_INCLUDE_EXTENSION_H",
        f"-D_GLIBCXX_USE_CXX11_ABI={abi}",
        f"-I{INCLUDE}", f"-I{py_inc}",
        *[f"-I{p}" for p in incs],
        os.path.join(CSRC, "binding.cpp"),
        "-o", tmp,
        *[f"-L{p}" for p in libdirs],
        f"-L{OUT_DIR}",
        "-l:" + HIP_LIB_NAME,
        "-lc10", "-ltorch", "-ltorch_cpu", "-ltorch_python", "-lc10_hip", "-ltorch_hip",
        "-Wl,-rpath,$ORIGIN",
        "-Wno-deprecated-declarations",
    ]
    _run(cmd, verbose)
    os.replace(tmp, out)
    return out


def build(verbose: bool = False) -> None:
    os.makedirs(OUT_DIR, exist_ok=True)
    build_hip_lib(verbose)
    build_binding(verbose)


if __name__ == "__main__":
    build(verbose="-q" not in sys.argv)
