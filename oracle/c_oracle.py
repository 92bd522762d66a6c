"""ctypes binding of the C oracle (oracle/kf_oracle.c).  TEST INFRASTRUCTURE ONLY."""

from __future__ import annotations

import ctypes
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libkf_oracle.so"

_lib = None


def build() -> Path:
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        lib = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.c_void_p
        I = ctypes.c_int
        lib.kfo_f32_to_f16.restype = ctypes.c_uint16
        lib.kfo_f32_to_f16.argtypes = [ctypes.c_float]
        lib.kfo_f16_to_f32.restype = ctypes.c_float
        lib.kfo_f16_to_f32.argtypes = [ctypes.c_uint16]
        lib.kfo_pack.argtypes = [P, I, I, P]
        lib.kfo_unpack.argtypes = [P, I, I, P]
        lib.kfo_lcg_workload.argtypes = [I, I, I, P, I, P, P, P, P]
        lib.kfo_dequant_fp16.argtypes = [P, P, I, I, I, P]
        lib.kfo_ref_f64.argtypes = [P, P, P, I, I, I, I, P]
        lib.kfo_max_rel_err_f16.restype = ctypes.c_double
        lib.kfo_max_rel_err_f16.argtypes = [P, P, ctypes.c_size_t]
        _lib = lib
    return _lib


def _p(a: np.ndarray):
    return a.ctypes.data_as(ctypes.c_void_p)


def f32_to_f16_bits(values) -> np.ndarray:
    lib = load()
    vals = np.asarray(values, dtype=np.float32).ravel()
    return np.array([lib.kfo_f32_to_f16(float(v)) for v in vals], dtype=np.uint16)


def pack(q: np.ndarray) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.int8)
    n, k = q.shape
    out = np.zeros((n, k // 8), dtype=np.int32)
    load().kfo_pack(_p(q), n, k, _p(out))
    return out


def unpack(packed: np.ndarray) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    n, kw = packed.shape
    out = np.zeros((n, kw * 8), dtype=np.int8)
    load().kfo_unpack(_p(packed), n, kw * 8, _p(out))
    return out


def lcg_workload(group: int, n: int = 128, k: int = 1024, ms=(1, 3, 8, 9, 16, 17, 33, 64, 65)):
    ms_arr = np.array(ms, dtype=np.int32)
    q = np.zeros((n, k), dtype=np.int8)
    scales = np.zeros((n, k // group), dtype=np.uint16)
    packed = np.zeros((n, k // 8), dtype=np.int32)
    xcat = np.zeros(int(ms_arr.sum()) * k, dtype=np.uint16)
    load().kfo_lcg_workload(group, n, k, _p(ms_arr), len(ms_arr), _p(q), _p(scales), _p(packed), _p(xcat))
    xs, off = {}, 0
    for m in ms:
        xs[m] = xcat[off:off + m * k].view(np.float16).reshape(m, k)
        off += m * k
    return q, scales.view(np.float16), packed, xs


def dequant_fp16(packed: np.ndarray, scales: np.ndarray, group: int) -> np.ndarray:
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    sc = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16)
    n, kw = packed.shape
    out = np.zeros((n, kw * 8), dtype=np.uint16)
    load().kfo_dequant_fp16(_p(packed), _p(sc), n, kw * 8, group, _p(out))
    return out.view(np.float16)


def ref_f64(x16: np.ndarray, packed: np.ndarray, scales: np.ndarray, group: int) -> np.ndarray:
    x = np.ascontiguousarray(x16, dtype=np.float16).view(np.uint16)
    packed = np.ascontiguousarray(packed, dtype=np.int32)
    sc = np.ascontiguousarray(scales, dtype=np.float16).view(np.uint16)
    m, k = x.shape
    n = packed.shape[0]
    y = np.zeros((m, n), dtype=np.float64)
    load().kfo_ref_f64(_p(x), _p(packed), _p(sc), m, n, k, group, _p(y))
    return y


def max_rel_err_f16(y16: np.ndarray, ref: np.ndarray) -> float:
    """kfo_max_rel_err_f16: the native check's pass-rule ratio of fp16 outputs against a float64 ref."""
    y = np.ascontiguousarray(y16, dtype=np.float16).view(np.uint16).ravel()
    r = np.ascontiguousarray(ref, dtype=np.float64).ravel()
    if y.size != r.size:
        raise ValueError("max_rel_err_f16: sizes differ")
    return float(load().kfo_max_rel_err_f16(_p(y), _p(r), y.size))
