"""Generated-code checks of the forward kernel's load waits (CPU only: hipcc
cross-compiles the head_dim-64 instances to gfx950 assembly).

The K/V tiles reach LDS through direct-to-LDS loads, which the vmcnt counter
tracks in issue order.  A workgroup barrier after such loads waits for all but
the wave's newest N of them (``barrier_after_loads<N>`` in
csrc/fa_kernel_common.h): N = 0 drains everything, N > 0 keeps the next tiles'
loads in flight.  These tests pin, in the instructions the compiler emits,
that the partial waits survive -- a workgroup fence in front of ``s_barrier``
(as ``__syncthreads()`` has) makes the compiler drain vmcnt to 0 there, and
the pipelining they were written for silently disappears:

* the prologue of a head_dim-64 instance waits only for the loads up to K_0's
  (vmcnt 4: two tiles of two 1 KB segments per wave still in flight), both in
  the 4-wave instance and in the 256-row one;
* the 256-row head_dim-64 instance (three K/V stages) ends each step of its
  main loop at a barrier that waits for all but the step's own two loads
  (vmcnt 2), never for all of them.
"""
import collections
import os
import re
import shutil
import subprocess
import sys
import tempfile

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(REPO, "flash-attention-sm75-register-fused_amd")
sys.path.insert(0, PKG)
import build_native  # noqa: E402

HIPCC = os.path.join(build_native.ROCM, "bin", "hipcc")

# Instance names: fa_fwd_kernel<D=64, CAUSAL=false, KV_SAME_STRIDE=true, WAVES,
# MASK_MODE=0, KSPLIT=false, BF16=false, ROWSUM=false, DYN=false>.
W8 = "fa_fwd_kernelILi64ELb0ELb1ELi8ELi0ELb0ELb0ELb0ELb0E"
W4 = "fa_fwd_kernelILi64ELb0ELb1ELi4ELi0ELb0ELb0ELb0ELb0E"
AFTER_K0 = 4   # prologue: K_1 and V_0 (4 waves) or K_1, K_2 / V_0, V_1 (split roles) in flight
LPW = 2        # direct loads per wave and step, 256-row head_dim-64 instance
STEP_MFMAS = 16


@pytest.fixture(scope="module")
def asm():
    if not os.path.exists(HIPCC):
        pytest.skip("hipcc not available")
    out = {}
    tmp = tempfile.mkdtemp(prefix="fa_codegen_")
    try:
        procs = {}
        for src in ("fa_fwd_d64.hip", "fa_fwd_d64_w8.hip"):
            dst = os.path.join(tmp, src + ".s")
            cmd = [HIPCC, *build_native.HIPCC_FLAGS, f"-I{build_native.INCLUDE}", f"-I{build_native.CSRC}",
                   "--cuda-device-only", "-S", os.path.join(build_native.CSRC, src), "-o", dst]
            procs[src] = (subprocess.Popen(cmd, stdout=subprocess.PIPE, stderr=subprocess.STDOUT, text=True), dst)
        for src, (p, dst) in procs.items():
            log, _ = p.communicate(timeout=600)
            assert p.returncode == 0, log
            out[src] = open(dst).read()
    finally:
        shutil.rmtree(tmp, ignore_errors=True)
    return out


def function_body(text, mangled_part):
    names = [m.group(1) for m in re.finditer(r"\n(_ZN2fa\S+):", text)]
    hits = [n for n in names if mangled_part in n]
    assert len(hits) == 1, (mangled_part, hits)
    body = text[text.index("\n" + hits[0] + ":"):]
    return body[:body.index(".Lfunc_end")].split("\n")


def waits_before_barriers(lines, lo=0, hi=None):
    """The s_waitcnt directly in front of each s_barrier of lines[lo:hi]."""
    hi = len(lines) if hi is None else hi
    found = []
    for j in range(lo, hi):
        if lines[j].strip().startswith("s_barrier"):
            k = j - 1
            # skip blank lines and comments (the empty asm statements around
            # the barrier leave ;;#ASMSTART / ;;#ASMEND markers)
            while k >= lo and (not lines[k].strip() or lines[k].strip().startswith(";")):
                k -= 1
            found.append(lines[k].strip() if lines[k].strip().startswith("s_waitcnt") else "")
    return found


def main_loop(lines, mfmas):
    """(start, end) of the loop whose body holds `mfmas` MFMAs (a backward branch)."""
    labels = {m.group(1): j for j, l in enumerate(lines) for m in [re.match(r"^(\.LBB\w+):", l)] if m}
    loops = []
    for j, l in enumerate(lines):
        m = re.search(r"s_c?branch\w*\s+(\.LBB\w+)", l)
        if m and m.group(1) in labels and labels[m.group(1)] < j:
            a = labels[m.group(1)]
            if sum("v_mfma" in lines[k] for k in range(a, j)) == mfmas:
                loops.append((a, j))
    assert len(loops) == 1, loops
    return loops[0]


def vmcnt(wait):
    m = re.search(r"vmcnt\((\d+)\)", wait)
    return int(m.group(1)) if m else None


def test_prologue_waits_only_for_k0(asm):
    for src, inst in (("fa_fwd_d64.hip", W4), ("fa_fwd_d64_w8.hip", W8)):
        waits = waits_before_barriers(function_body(asm[src], inst))
        counts = collections.Counter(vmcnt(w) for w in waits)
        assert counts[AFTER_K0] == 1, (src, waits)


def test_three_stage_loop_keeps_next_tiles_in_flight(asm):
    lines = function_body(asm["fa_fwd_d64_w8.hip"], W8)
    lo, hi = main_loop(lines, 3 * STEP_MFMAS)  # the loop is unrolled by its three stages
    waits = waits_before_barriers(lines, lo, hi)
    assert len(waits) == 3, waits
    assert all(vmcnt(w) == LPW and "lgkmcnt(0)" in w for w in waits), waits
