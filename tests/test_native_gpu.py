"""The torch-free native check (tests/native/kf_native_check.cpp) on the GPU.

A host C++ program over the C ABI with the reference's LCG workload and a double-precision
reference (the counterpart of the reference's csrc/micro/sanitize_gemm.cu), run as a child
process: plainly, and built with AddressSanitizer + UBSan on its host code.
"""

from __future__ import annotations

import os
import subprocess
from pathlib import Path

import pytest

NATIVE = Path(__file__).resolve().parent / "native"


def _run(exe: Path) -> subprocess.CompletedProcess:
    if not exe.exists():
        pytest.fail(f"{exe.name} is not built (run __graft_entry__.build())")
    env = dict(os.environ, ASAN_OPTIONS="detect_leaks=0", UBSAN_OPTIONS="print_stacktrace=1:halt_on_error=1")
    return subprocess.run([str(exe)], capture_output=True, text=True, timeout=120, env=env)


@pytest.mark.gpu
@pytest.mark.parametrize("variant", ["kf_native_check", "kf_native_check_asan"])
def test_native_check(variant):
    r = _run(NATIVE / variant)
    print(r.stdout[-4000:], r.stderr[-4000:])
    assert r.returncode == 0, r.stdout[-2000:] + r.stderr[-2000:]
    assert "OK (0 failures)" in r.stdout
    # Both groups: the GEMM at M in {1, 3, 8, 9, 16, 17, 33, 64, 65}, the GEMV at the three M <= 8,
    # and the fused decode GEMV's two prologues.
    assert r.stdout.count(" err=") == 2 * (9 + 3 + 2)
    assert r.stdout.count("fused residual bit-exact=1") == 2
    assert r.stdout.count("v bit-exact=1 cache=1") == 2


def test_native_check_links():
    """Both binaries exist and every shared library they need resolves (no GPU needed)."""
    for variant in ("kf_native_check", "kf_native_check_asan"):
        exe = NATIVE / variant
        assert exe.exists(), f"{variant} is not built"
        out = subprocess.run(["ldd", str(exe)], capture_output=True, text=True, check=True).stdout
        assert "not found" not in out, out
        assert "libkf_int4.so" in out
