"""CPU oracle of the INT4 weight-only linear path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
anything under oracle/, and only as the checker (or, for cpu_baseline, as the
timed CPU restatement of the reference's FP32 dequant+matmul).  The product
package never imports it.

  int4_oracle.py   numpy restatement (quantize, pack/unpack, dequantize, FP32 reference)
  kf_oracle.c      C restatement of the reference's torch-free LCG workload
  c_oracle.py      ctypes binding of libkf_oracle.so (built by oracle/Makefile)
  cpu_baseline.py  the reference's CPU FP32 dequant + matmul in torch (bench.py's cpu_baseline leg)

Every function is pinned in tests/test_oracle.py (KATs, exact rational arithmetic, brute force,
the C restatement; quantization_error on a crafted weight with exact errors).  The pass rule
itself, max_rel_err (numpy) and kfo_max_rel_err_f16 (C, used by the native check), is pinned by
hand-computed dyadic cases that each plausible misreading fails: a per-element ratio, a mean, a
missing abs, a scale taken from out, a per-row scale, a dropped NaN, an all-zero ref, a shape
mismatch.  No function is left "parity unpinned".
"""
