"""CPU oracle of the attention forward -- TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the math of the reference's own parity path
(reference src/reference/attention_ref.py:10-45 and
src/reference/correctness.py:8-37) so that the GPU kernels can be checked
against it.  It is never part of the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker (or, for the baseline, as the timed CPU
implementation of the reference algorithm).  The product path
(``flash_attention_sm75``) never imports it and has no CPU fallback.

Modules
  attention_ref  numpy restatement (fp32, the reference's op order), fp64
                 brute force, row log-sum-exp, chunked runner for large shapes,
                 the correctness metric, and a torch-CPU restatement used as
                 the timed CPU baseline.
  c_oracle       ctypes loader for ``attention_oracle.c``: an independent
                 long-double/double two-pass C statement of the same math and
                 an fp32 tiled online-softmax statement of the reference's
                 scalar kernel (src/kernels/flash_attention_forward.cu:48-163).

How each function is pinned (there are no golden data files in the
reference): see the docstrings; every function is checked in
tests/test_oracle.py against an fp64 brute force, closed forms and invariants
(causal row 0 equals V[0]; constant V gives V; key permutation invariance;
scale -> 0 gives the mean of visible V rows; a single key gives V; GQA equals
explicit repeat_interleave), and against the reference's own input generators
(glibc rand() streams of fused/src/flash_mha_v2.cu:34-36,608-613 and
fused/src/test_warp_softmax.cu:151-154).
"""
