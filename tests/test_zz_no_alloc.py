"""kf_int4_gemm_noalloc, the GEMM entry point that allocates nothing, through the C ABI.

Its split-K partials live in the library's per-GPU scratch array instead of a caller workspace.
Checked against kf_int4_gemm (same plan and kernels, a torch-allocated workspace) bit for bit,
on two calls in a row with split-K where the second problem is smaller (so stale partials of the
first call sit in the scratch), on plans without split-K (tiled and skinny kernels), and on the
refusal of a plan whose partials exceed the scratch (no launch).
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kernelforge import _lib
from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu
DEV = "cuda"
G = 128


def _inputs(m, n, k, seed):
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    packed, scales = o.quantize_weight(w, G)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    return (torch.from_numpy(x).to(DEV), torch.from_numpy(packed).to(DEV), torch.from_numpy(scales).to(DEV),
            (x, packed, scales))


def _plan(m, n, k):
    """(kernel, splits, workspace bytes) of kf_int4_gemm's plan on this device."""
    lib = _lib.load()
    kernel, num, splits, bm, bn = (ctypes.c_int() for _ in range(5))
    _lib.check(lib.kf_int4_gemm_plan(m, n, k, G, ctypes.byref(kernel), ctypes.byref(num), ctypes.byref(splits),
                                     ctypes.byref(bm), ctypes.byref(bn)), "plan")
    return kernel.value, splits.value, lib.kf_int4_gemm_workspace_bytes(m, n, k, G)


def _stream():
    return torch.cuda.current_stream().cuda_stream


def _with_workspace(x, p, s, m, n, k):
    lib = _lib.load()
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    ws_bytes = lib.kf_int4_gemm_workspace_bytes(m, n, k, G)
    ws = torch.empty(max(ws_bytes, 4) // 4, dtype=torch.float32, device=DEV)
    _lib.check(lib.kf_int4_gemm(x.data_ptr(), p.data_ptr(), s.data_ptr(), y.data_ptr(),
                                ws.data_ptr() if ws_bytes else None, ws_bytes, m, n, k, G, _stream()), "gemm")
    return y


def _noalloc(x, p, s, m, n, k):
    lib = _lib.load()
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    _lib.check(lib.kf_int4_gemm_noalloc(x.data_ptr(), p.data_ptr(), s.data_ptr(), y.data_ptr(), m, n, k, G,
                                        _stream()), "gemm_noalloc")
    return y


# (M, N, K): a split-K plan (TinyLlama down at M = 64), then a smaller split-K plan picked from
# ragged shapes; then plans without split-K.
FIRST = (64, 2048, 5632)
SMALLER = [(33, 320, 4224), (33, 64, 1152), (65, 192, 4160), (33, 640, 8960), (47, 704, 5120), (32, 1536, 8960)]


def test_two_calls_in_a_row_match_the_workspace_entry_point():
    big = _plan(*FIRST)
    assert big[1] > 1 and 0 < big[2] <= _lib.KF_NOALLOC_SCRATCH_BYTES, f"expected a split-K plan, got {big}"
    second = [c for c in SMALLER if _plan(*c)[1] > 1 and 0 < _plan(*c)[2] < big[2] and c[0] * c[1] < FIRST[0] * FIRST[1]]
    assert second, "no smaller split-K plan among the candidates"
    SECOND = second[0]
    for seed, (m, n, k) in enumerate((FIRST, SECOND)):
        x, p, s, host = _inputs(m, n, k, 100 + seed)
        y = _noalloc(x, p, s, m, n, k)
        ref = _with_workspace(x, p, s, m, n, k)
        torch.cuda.synchronize()
        print(f"noalloc M={m} N={n} K={k}: plan {_plan(m, n, k)}", flush=True)
        assert torch.equal(y, ref), f"M={m} N={n} K={k}: noalloc differs from kf_int4_gemm"
        assert o.max_rel_err(y.float().cpu().numpy(), o.linear_ref_fp32(host[0], host[1], host[2], G)) <= 2e-3


@pytest.mark.parametrize("m,n,k", [(2048, 5632, 2048), (4, 2048, 5632), (1, 256, 2048)])
def test_plans_without_split_k(m, n, k):
    assert _plan(m, n, k)[2] == 0
    x, p, s, _ = _inputs(m, n, k, 7)
    assert torch.equal(_noalloc(x, p, s, m, n, k), _with_workspace(x, p, s, m, n, k))


def test_refuses_a_plan_larger_than_the_scratch():
    """A long-K problem on few tiles splits K many ways: its partials exceed the scratch, so the
    entry point returns KF_ERR_WORKSPACE before launching (y stays untouched)."""
    # On 256 CUs: 128 x 128 tiles split 3 ways (60 MiB of partials), 5 ways (60 MiB), 7 ways (63 MiB).
    for m, n, k in [(2048, 2560, 16384), (1536, 2048, 32768), (1536, 1536, 65536)]:
        if _plan(m, n, k)[2] > _lib.KF_NOALLOC_SCRATCH_BYTES:
            break
    else:
        pytest.skip("no candidate plan exceeds the scratch on this device")
    x = torch.zeros(m, k, dtype=torch.float16, device=DEV)
    p = torch.zeros(n, k // 8, dtype=torch.int32, device=DEV)
    s = torch.ones(n, k // G, dtype=torch.float16, device=DEV)
    y = torch.full((m, n), 7.0, dtype=torch.float16, device=DEV)
    lib = _lib.load()
    st = lib.kf_int4_gemm_noalloc(x.data_ptr(), p.data_ptr(), s.data_ptr(), y.data_ptr(), m, n, k, G, _stream())
    assert st == _lib.KF_ERR_WORKSPACE and "scratch" in _lib.last_error()
    torch.cuda.synchronize()
    assert bool((y == 7.0).all())
