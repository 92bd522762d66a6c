"""The C-ABI library: it loads, exports exactly what include/kf_int4.h declares,
and rejects bad arguments before any GPU work (no compute calls here)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np
import pytest

from kernelforge import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "kf_int4.h"
MAX_ROWS = (1 << 25) - 64  # KF_MAX_ROWS in the header


def test_row_limit_matches_header():
    assert re.search(r"#define KF_MAX_ROWS \(\(1 << 25\) - 64\)", HEADER.read_text())


def _declared_symbols() -> set[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return set(re.findall(r"\b(kf_[a-z0-9_]+)\s*\(", text))


def test_header_and_binding_agree():
    assert _declared_symbols() == set(_lib.SIGNATURES)


def test_library_loads_and_exports_every_declared_symbol():
    lib = _lib.load()
    for name in _declared_symbols():
        assert hasattr(lib, name), name
    assert lib.kf_abi_version() == _lib.ABI_VERSION


def _err(status, match):
    assert status != 0
    assert re.search(match, _lib.last_error()), _lib.last_error()


def test_gemv_argument_errors_without_gpu():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)  # never dereferenced: validation fails first
    _err(lib.kf_int4_gemv(None, p, p, p, 1, 64, 256, 128, None), "non-null")
    _err(lib.kf_int4_gemv(p, p, p, p, 1, 64, 200, 128, None), "not a multiple of group_size")
    _err(lib.kf_int4_gemv(p, p, p, p, 1, 64, 256, 32, None), "group_size")
    _err(lib.kf_int4_gemv(p, p, p, p, 9, 64, 256, 128, None), r"M in \[1, 8\]")
    _err(lib.kf_int4_gemv(p, p, p, p, 0, 64, 256, 128, None), "positive")
    # empty tensors have null data pointers: their sizes are what the error names
    _err(lib.kf_int4_gemv(p, None, None, None, 1, 0, 256, 128, None), "positive, got M=1 N=0")
    _err(lib.kf_int4_gemm(None, p, p, None, None, 0, 0, 128, 256, 128, None), "positive, got M=0")
    _err(lib.kf_int4_gemv(ctypes.c_void_p(0x1002), p, p, p, 1, 64, 256, 128, None), "16-byte aligned")
    with pytest.raises(ValueError, match=r"M in \[1, 8\]"):
        _lib.check(lib.kf_int4_gemv(p, p, p, p, 9, 64, 256, 128, None), "int4_gemv")


def test_grouped_gemv_argument_errors_without_gpu():
    lib = _lib.load()
    good = _lib.GemvProblem(0x1000, 0x1000, 0x1000, 0x1000, 64, 256)
    bad_k = _lib.GemvProblem(0x1000, 0x1000, 0x1000, 0x1000, 64, 200)
    arr = (_lib.GemvProblem * 9)(*([good] * 9))
    _err(lib.kf_int4_gemv_grouped(None, 1, 1, 128, None), "non-null")
    _err(lib.kf_int4_gemv_grouped(arr, 0, 1, 128, None), r"count must be in \[1, 8\]")
    _err(lib.kf_int4_gemv_grouped(arr, 9, 1, 128, None), r"count must be in \[1, 8\]")
    _err(lib.kf_int4_gemv_grouped(arr, 2, 9, 128, None), r"M in \[1, 8\]")
    mixed = (_lib.GemvProblem * 2)(good, bad_k)
    _err(lib.kf_int4_gemv_grouped(mixed, 2, 1, 128, None), "problem 1: K=200 is not a multiple of group_size")
    half = _lib.GemvProblem(0x1000, 0x1000, 0x1000, 0x1000, MAX_ROWS // 2 + 64, 256)
    _err(lib.kf_int4_gemv_grouped((_lib.GemvProblem * 2)(half, half), 2, 1, 128, None),
         f"rows in total, more than the {MAX_ROWS}")


def test_row_limit_without_gpu():
    """N beyond KF_MAX_ROWS (a grid past 2^31 work-items at one row per wavefront) is refused
    before any launch, by the GEMV and the GEMM alike."""
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    _err(lib.kf_int4_gemv(p, p, p, p, 1, MAX_ROWS + 1, 256, 128, None), f"exceeds the {MAX_ROWS} rows")
    _err(lib.kf_int4_gemm(p, p, p, p, None, 0, 16, MAX_ROWS + 64, 256, 128, None), f"exceeds the {MAX_ROWS} rows")
    with pytest.raises(ValueError, match="exceeds"):
        _lib.check(lib.kf_int4_gemv(p, p, p, p, 1, MAX_ROWS + 1, 256, 128, None), "int4_gemv")


def test_gemm_argument_errors_without_gpu():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    _err(lib.kf_int4_gemm(p, p, p, p, None, 0, 16, 100, 256, 128, None), "multiple of 64")
    _err(lib.kf_int4_gemm(p, p, None, p, None, 0, 16, 128, 256, 128, None), "non-null")
    _err(lib.kf_int4_gemm(p, p, p, p, None, 0, 16, 128, 320, 128, None), "not a multiple of group_size")
    y2 = ctypes.c_void_p(0x1002)  # 2-byte aligned: enough for the GEMV, not for the GEMM's vector stores
    _err(lib.kf_int4_gemm(p, p, p, y2, None, 0, 16, 128, 256, 128, None), "y to be 16-byte aligned")
    _err(lib.kf_int4_gemm_noalloc(p, p, p, y2, 16, 128, 256, 128, None), "y to be 16-byte aligned")
    _err(lib.kf_int4_gemm_mfma16(p, p, p, p, p, y2, None, 0, 16, 128, 256, 128, None), "y to be 16-byte aligned")
    _err(lib.kf_int4_dequant_fp16(None, p, p, 4, 256, 128, None), "non-null")
    _err(lib.kf_bw_copy(p, p, 17, 0, None), "multiple of 16")
    assert lib.kf_int4_gemm_workspace_bytes(0, 64, 256, 128) == 0


def test_decode_argmax_step_argument_errors_without_gpu():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    _err(lib.kf_decode_argmax_step(None, 16, p, p, p, 8, None, None), "non-null")
    _err(lib.kf_decode_argmax_step(p, 16, p, None, p, 8, None, None), "non-null")
    _err(lib.kf_decode_argmax_step(p, 0, p, p, p, 8, None, None), "positive")
    _err(lib.kf_decode_argmax_step(p, 16, p, p, p, 0, None, None), "positive")
    _err(lib.kf_decode_argmax_step(ctypes.c_void_p(0x1001), 16, p, p, p, 8, None, None), "2-byte aligned")
    _err(lib.kf_decode_argmax_step(p, 16, p, p, p, 8, ctypes.c_void_p(0x1003), None), "2-byte aligned")
    _err(lib.kf_decode_argmax_step(p, 16, ctypes.c_void_p(0x1004), p, p, 8, None, None), "8-byte aligned")


def test_fused_gemv_argument_errors_without_gpu():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    eps = ctypes.c_float(1e-5)
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 2, 64, 256, 128, 0, None, eps, None, None), "M = 1")
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 1, 64, 256, 128, 3, None, eps, None, None), "prologue must be")
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 1, 64, 256, 128, _lib.KF_PROLOGUE_RMSNORM, None, eps, None, None),
         "aux input must be non-null")
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 1, 64, 256, 128, _lib.KF_PROLOGUE_SWIGLU, ctypes.c_void_p(0x1008), eps,
                                None, None), "16-byte aligned")
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 1, 64, 256, 128, _lib.KF_PROLOGUE_RMSNORM, p, ctypes.c_float(-1.0),
                                None, None), "eps must be finite")
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 1, 64, 256, 128, 0, None, eps, ctypes.c_void_p(0x1001), None),
         "residual must be 2-byte aligned")
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 1, 64, 10240 + 128, 128, 0, None, eps, None, None), "K <= 10240")
    _err(lib.kf_int4_gemv_fused(p, p, p, p, 1, 64, 200, 128, 0, None, eps, None, None), "not a multiple of group_size")


def test_fused_constants_match_header():
    text = HEADER.read_text()
    for name in ("KF_PROLOGUE_NONE", "KF_PROLOGUE_RMSNORM", "KF_PROLOGUE_SWIGLU", "KF_GEMV_FUSED_MAX_K"):
        m = re.search(rf"#define {name} (\d+)", text)
        assert m and int(m.group(1)) == getattr(_lib, name), name



def test_qkv_rope_argument_errors_without_gpu():
    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    eps = ctypes.c_float(1e-5)
    rc = _lib.RopeCache(0x1000, 0x1000, 0x1000, 0x1000, 0x1000, 32, 4, 64, 160)
    _err(lib.kf_int4_gemv_qkv_rope(p, p, p, p, 2560, 2048, 128, None, eps, None, None), "rope must be non-null")
    _err(lib.kf_int4_gemv_qkv_rope(p, p, p, p, 2048, 2048, 128, None, eps, ctypes.byref(rc), None),
         r"not \(heads \+ 2 kv_heads\) \* head_dim")
    bad = _lib.RopeCache(0x1000, 0x1000, 0x1004, 0x1000, 0x1000, 32, 4, 64, 160)
    _err(lib.kf_int4_gemv_qkv_rope(p, p, p, p, 2560, 2048, 128, None, eps, ctypes.byref(bad), None), "8-byte")
    odd = _lib.RopeCache(0x1000, 0x1000, 0x1000, 0x1000, 0x1000, 32, 4, 63, 160)
    _err(lib.kf_int4_gemv_qkv_rope(p, p, p, p, 2520, 2048, 128, None, eps, ctypes.byref(odd), None), "even head_dim")
    nul = _lib.RopeCache(0x1000, 0, 0x1000, 0x1000, 0x1000, 32, 4, 64, 160)
    _err(lib.kf_int4_gemv_qkv_rope(p, p, p, p, 2560, 2048, 128, None, eps, ctypes.byref(nul), None), "non-null")
    _err(lib.kf_int4_gemv_qkv_rope(p, p, p, p, 2560, 10240 + 128, 128, None, eps, ctypes.byref(rc), None),
         "K <= 10240")


# ---------------------------------------------------------------------------
# GEMV launch plan (host code: kf_int4_gemv_plan with an explicit CU count)
# ---------------------------------------------------------------------------

QWEN_SEVEN = [(1536, 1536), (256, 1536), (256, 1536), (1536, 1536), (8960, 1536), (8960, 1536), (1536, 8960)]
TL_SEVEN = [(2048, 2048), (256, 2048), (256, 2048), (2048, 2048), (5632, 2048), (5632, 2048), (2048, 5632)]
CUS = 256  # MI355X
SLOTS = 32 * CUS  # 8 wavefronts per SIMD, 4 SIMDs per CU


def _entry_rows(entry: int) -> int:
    return 2 if entry == _lib.KF_GEMV_DEEP else (entry - _lib.KF_GEMV_FLAT if entry > _lib.KF_GEMV_FLAT else entry)


def _waves(shapes, rows, x_lds) -> int:
    total = 0
    for (n, _), entry in zip(shapes, rows):
        w = -(-n // _entry_rows(entry))
        total += -(-w // 4) * 4 if x_lds else w
    return total


def test_gemv_plan_constants_match_header():
    text = HEADER.read_text()
    for name in ("KF_GEMV_KERNEL_ROWS1", "KF_GEMV_KERNEL_ROWS2", "KF_GEMV_KERNEL_MIXED", "KF_GEMV_KERNEL_SHAPED",
                 "KF_GEMV_DEEP", "KF_GEMV_FLAT"):
        m = re.search(rf"#define {name} (\d+)", text)
        assert m and int(m.group(1)) == getattr(_lib, name), name


def test_gemv_plan_benchmarked_sets_without_gpu():
    """The plans behind the benchmark's two 7-linear steps (M = 1, 256 CUs)."""
    flat4 = _lib.KF_GEMV_FLAT + 4
    qwen = _lib.gemv_plan(1, QWEN_SEVEN, CUS)
    assert qwen["kernel"] == _lib.KF_GEMV_KERNEL_SHAPED and qwen["x_lds"] and qwen["unroll"] == 1
    assert qwen["rows"] == [flat4] * 6 + [_lib.KF_GEMV_DEEP]  # K = 1536: 4 rows in 3 full loads; down: deep
    assert _waves(QWEN_SEVEN, qwen["rows"], True) == 6144 <= SLOTS
    tl = _lib.gemv_plan(1, TL_SEVEN, CUS)
    # deep rows (two per wavefront, like plain rows) leave 8,960 wavefronts for 8,192 slots: the
    # plan keeps plain two-row down and gives gate three rows
    assert tl["kernel"] == _lib.KF_GEMV_KERNEL_MIXED and tl["rows"] == [2, 2, 2, 2, 3, 2, 2]
    assert _waves(TL_SEVEN, tl["rows"], True) == 8024 <= SLOTS


def test_gemv_plan_rules_without_gpu():
    flat2 = _lib.KF_GEMV_FLAT + 2
    # many K = 1024 rows: flat two-row problems go to three rows, largest first, until the grid fits
    heavy = [(9001, 1024), (8999, 1024), (4099, 1024), (257, 1024), (3, 1024), (1, 1024)]
    p = _lib.gemv_plan(1, heavy, CUS)
    assert p["kernel"] == _lib.KF_GEMV_KERNEL_SHAPED and p["rows"] == [3, 3, 3, flat2, flat2, flat2]
    assert _waves(heavy, p["rows"], True) <= SLOTS
    # flat and deep rows need M = 1 and x in LDS
    for m in (2, 5, 8):
        q = _lib.gemv_plan(m, QWEN_SEVEN, CUS)
        assert all(r <= 3 for r in q["rows"]) and q["kernel"] != _lib.KF_GEMV_KERNEL_SHAPED
    # single problems: one row per wavefront below 8 wavefronts per CU, else two
    assert _lib.gemv_plan(1, [(2048, 2048)], CUS)["kernel"] == _lib.KF_GEMV_KERNEL_ROWS1
    assert _lib.gemv_plan(1, [(5632, 2048)], CUS)["kernel"] == _lib.KF_GEMV_KERNEL_ROWS2
    # K = 1536 / 1024 rows in a small launch keep one row per wavefront (no flat rows)
    small = _lib.gemv_plan(1, [(256, 1536), (256, 1024)], CUS)
    assert small["kernel"] == _lib.KF_GEMV_KERNEL_ROWS1 and small["rows"] == [1, 1]


def test_gemv_plan_fits_one_round_without_gpu():
    """Random grouped launches at M = 1 and 2: whenever the plan leaves a two-row problem (plain
    or flat) it has found a grid that fits the 8,192 wave slots; deep rows appear only in grids
    that fit; flat rows only for K = 1024 / 1536."""
    rng = np.random.default_rng(7)
    for _ in range(300):
        count = int(rng.integers(2, 9))
        shapes = [(int(rng.integers(1, 12000)), int(rng.choice([512, 1024, 1536, 2048, 3072, 5632, 8960])))
                  for _ in range(count)]
        for m in (1, 2):
            p = _lib.gemv_plan(m, shapes, CUS)
            rows = p["rows"]
            if p["kernel"] in (_lib.KF_GEMV_KERNEL_MIXED, _lib.KF_GEMV_KERNEL_SHAPED):
                waves = _waves(shapes, rows, p["x_lds"])
                if any(r in (2, _lib.KF_GEMV_FLAT + 2) for r in rows) or _lib.KF_GEMV_DEEP in rows:
                    assert waves <= SLOTS, (m, shapes, p)
            for (n, k), r in zip(shapes, rows):
                if r > _lib.KF_GEMV_FLAT:
                    assert m == 1 and k in (1024, 1536) and r == _lib.KF_GEMV_FLAT + (4 if k == 1536 else 2)
                if r == _lib.KF_GEMV_DEEP:
                    assert m == 1 and k > 2048


def test_gemv_plan_argument_errors_without_gpu():
    lib = _lib.load()
    one = (ctypes.c_int * 1)(64)
    k = (ctypes.c_int * 1)(256)
    _err(lib.kf_int4_gemv_plan(1, None, k, 1, CUS, None, None, None, None), "non-null")
    _err(lib.kf_int4_gemv_plan(1, one, k, 9, CUS, None, None, None, None), "count")
    _err(lib.kf_int4_gemv_plan(9, one, k, 1, CUS, None, None, None, None), r"M in \[1, 8\]")
    bad = (ctypes.c_int * 1)(200)
    _err(lib.kf_int4_gemv_plan(1, one, bad, 1, CUS, None, None, None, None), "multiple of 64")


def test_last_error_is_per_thread():
    """kf_last_error names the calling thread's own most recent failure: two threads that fail
    differently, interleaved, each read back their own message."""
    import threading

    lib = _lib.load()
    p = ctypes.c_void_p(0x1000)
    barrier = threading.Barrier(2)
    seen = {}

    def worker(name, call, want):
        barrier.wait()
        assert call() != 0
        barrier.wait()  # both threads have failed before either reads its message
        seen[name] = (_lib.last_error(), want)

    threads = [threading.Thread(target=worker, args=("group", lambda: lib.kf_int4_gemv(p, p, p, p, 1, 64, 256, 32, None),
                                                     "group_size")),
               threading.Thread(target=worker, args=("m", lambda: lib.kf_int4_gemv(p, p, p, p, 9, 64, 256, 128, None),
                                                     r"M in \[1, 8\]"))]
    for t in threads:
        t.start()
    for t in threads:
        t.join()
    assert set(seen) == {"group", "m"}
    for msg, want in seen.values():
        assert re.search(want, msg), msg
    assert not re.search(r"M in \[1, 8\]", seen["group"][0]) and "group_size" not in seen["m"][0]
