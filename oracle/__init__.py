"""CPU oracle of the INT4 weight-only linear path.  TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
anything under oracle/, and only as the checker (or, for cpu_baseline, as the
timed CPU restatement of the reference's FP32 dequant+matmul).  The product
package never imports it.

  int4_oracle.py   numpy restatement (quantize, pack/unpack, dequantize, FP32 reference)
  kf_oracle.c      C restatement of the reference's torch-free LCG workload
  c_oracle.py      ctypes binding of libkf_oracle.so (built by oracle/Makefile)

Parity of every function is pinned in tests/test_oracle.py; none is "parity unpinned".
"""
