"""ctypes binding of libkf_int4.so, the gfx950 HIP library behind kernelforge.ops.

The library exports a plain C ABI (include/kf_int4.h).  This module loads it
from the package directory, declares the signatures, and turns non-zero
status codes into Python exceptions.  There is no fallback: if the library is
missing or cannot be loaded, every op raises ImportError.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIB_PATH = Path(__file__).resolve().with_name("libkf_int4.so")
ABI_VERSION = 1

KF_OK = 0
KF_ERR_INVALID_ARG = 1
KF_ERR_UNSUPPORTED = 2
KF_ERR_WORKSPACE = 3
KF_ERR_HIP = 4
KF_PROLOGUE_NONE = 0
KF_PROLOGUE_RMSNORM = 1
KF_PROLOGUE_SWIGLU = 2
KF_GEMV_FUSED_MAX_K = 10240
KF_NOALLOC_SCRATCH_BYTES = 32 << 20
KF_GEMV_KERNEL_ROWS1, KF_GEMV_KERNEL_ROWS2, KF_GEMV_KERNEL_MIXED, KF_GEMV_KERNEL_SHAPED = 1, 2, 3, 4
KF_GEMV_DEEP = 8
KF_GEMV_FLAT = 16

GEMV_MAX_GROUP = 8


class GemvProblem(ctypes.Structure):
    """kf_gemv_problem of include/kf_int4.h."""

    _fields_ = [("x", ctypes.c_void_p), ("packed", ctypes.c_void_p), ("scales", ctypes.c_void_p),
                ("y", ctypes.c_void_p), ("N", ctypes.c_int), ("K", ctypes.c_int)]


# Every symbol include/kf_int4.h declares, with (restype, argtypes).
_VP, _I, _SZ = ctypes.c_void_p, ctypes.c_int, ctypes.c_size_t
_IP = ctypes.POINTER(ctypes.c_int)
class RopeCache(ctypes.Structure):
    """kf_rope_cache of include/kf_int4.h."""
    _fields_ = [("cos", ctypes.c_void_p), ("sin", ctypes.c_void_p), ("pos", ctypes.c_void_p),
                ("cache_k", ctypes.c_void_p), ("cache_v", ctypes.c_void_p), ("heads", ctypes.c_int),
                ("kv_heads", ctypes.c_int), ("head_dim", ctypes.c_int), ("max_seq", ctypes.c_int)]


SIGNATURES = {
    "kf_abi_version": (_I, []),
    "kf_last_error": (ctypes.c_char_p, []),
    "kf_int4_gemv": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP]),
    "kf_int4_gemv_grouped": (_I, [ctypes.POINTER(GemvProblem), _I, _I, _I, _VP]),
    "kf_int4_gemv_fused": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _I, _I, _VP, ctypes.c_float, _VP, _VP]),
    "kf_int4_gemv_qkv_rope": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _VP, ctypes.c_float, ctypes.POINTER(RopeCache),
                                   _VP]),
    "kf_int4_gemm_workspace_bytes": (_SZ, [_I, _I, _I, _I]),
    "kf_int4_gemm_plan": (_I, [_I, _I, _I, _I, _IP, _IP, _IP, _IP, _IP]),
    "kf_int4_gemv_plan": (_I, [_I, _IP, _IP, _I, _I, _IP, _IP, _IP, _IP]),
    "kf_int4_gemm": (_I, [_VP, _VP, _VP, _VP, _VP, _SZ, _I, _I, _I, _I, _VP]),
    "kf_int4_gemm_noalloc": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _I, _VP]),
    "kf_int4_mfma16_sizes": (_I, [_I, _I, _I, ctypes.POINTER(_SZ), ctypes.POINTER(_SZ)]),
    "kf_int4_reorder_mfma16": (_I, [_VP, _VP, _VP, _VP, _I, _I, _I, _VP]),
    "kf_int4_gemm_mfma16": (_I, [_VP, _VP, _VP, _VP, _VP, _VP, _VP, _SZ, _I, _I, _I, _I, _VP]),
    "kf_int4_dequant_fp16": (_I, [_VP, _VP, _VP, _I, _I, _I, _VP]),
    "kf_int4_quantize": (_I, [_VP, _I, _VP, _VP, _I, _I, _I, _VP]),
    "kf_bw_copy": (_I, [_VP, _VP, _SZ, _I, _VP]),
    "kf_bw_read": (_I, [_VP, _VP, _SZ, _I, _VP]),
    "kf_bw_write": (_I, [_VP, _SZ, _I, _VP]),
    "kf_bw_read_store": (_I, [_VP, _VP, _SZ, _I, _VP]),
    "kf_decode_argmax_step": (_I, [_VP, _I, _VP, _VP, _VP, _I, _VP, _VP]),
}

_lib: ctypes.CDLL | None = None
_load_error: Exception | None = None


def load() -> ctypes.CDLL:
    """Loads and type-annotates the library once; raises ImportError if it is unavailable."""
    global _lib, _load_error
    if _lib is not None:
        return _lib
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH.name} is not built (expected at {LIB_PATH}). "
                          "Build it with `python kernel-forge_amd/kernelforge/build.py` (hipcc, gfx950).")
    try:
        lib = ctypes.CDLL(str(LIB_PATH))
    except OSError as exc:  # missing HIP runtime, wrong architecture, ...
        _load_error = exc
        raise ImportError(f"cannot load {LIB_PATH}: {exc}") from exc
    for name, (restype, argtypes) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    version = lib.kf_abi_version()
    if version != ABI_VERSION:
        raise ImportError(f"{LIB_PATH.name} has ABI version {version}, expected {ABI_VERSION}; rebuild it")
    _lib = lib
    return lib


def last_error() -> str:
    msg = load().kf_last_error()
    return msg.decode("utf-8", "replace") if msg else ""


def check(status: int, what: str) -> None:
    """Raises for a non-zero status: ValueError for argument errors, RuntimeError otherwise."""
    if status == KF_OK:
        return
    msg = f"{what}: {last_error()}"
    if status in (KF_ERR_INVALID_ARG, KF_ERR_UNSUPPORTED):
        raise ValueError(msg)
    raise RuntimeError(msg)


def gemv_plan(m: int, shapes: list[tuple[int, int]], cu_count: int = 0) -> dict:
    """The GEMV launch plan (kf_int4_gemv_plan) for M and [(N, K), ...]: the kernel kind, each
    problem's rows entry (1-3 rows per wavefront, KF_GEMV_FLAT + F or KF_GEMV_DEEP), the unroll and
    whether x is staged in LDS.  Host-only when cu_count > 0 (no GPU needed)."""
    lib = load()
    count = len(shapes)
    ns = (ctypes.c_int * count)(*[n for n, _ in shapes])
    ks = (ctypes.c_int * count)(*[k for _, k in shapes])
    kernel, unroll, x_lds = ctypes.c_int(), ctypes.c_int(), ctypes.c_int()
    rows = (ctypes.c_int * count)()
    check(lib.kf_int4_gemv_plan(m, ns, ks, count, cu_count, ctypes.byref(kernel), rows, ctypes.byref(unroll),
                                ctypes.byref(x_lds)), "int4_gemv_plan")
    return {"kernel": kernel.value, "rows": list(rows), "unroll": unroll.value, "x_lds": bool(x_lds.value)}
