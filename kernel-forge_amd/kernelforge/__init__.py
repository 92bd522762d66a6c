"""KernelForge INT4 weight-only linear, MI355X-native (gfx950 HIP kernels behind a C ABI).

Submodules:
  quantize  the packed INT4 format (producer, reference kernelforge/quantize.py)
  ops       int4_gemv / int4_gemm / int4_matmul / int4_linear + torch.library op
  modules   KFLinearInt4 and quantize_linears_
  _lib      ctypes binding of libkf_int4.so
  build     hipcc build of libkf_int4.so
"""

__version__ = "0.3.0"
__all__ = ["quantize", "ops", "modules"]
