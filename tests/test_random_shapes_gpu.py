"""Seeded random shapes through the GEMV, the grouped GEMV and the GEMM, against the CPU oracle.

The fixed shape lists elsewhere name the benchmark layers and hand-picked edges; these cases are
drawn from a fixed seed so that the launch plans meet shapes nobody chose: ragged N at every M,
K from 64 to 6,144 (flat rows at K = 1,024 / 1,536, deep and multi-pass rows past 2,048), groups of
2-8 problems with different K in one launch (three-row, flat and deep mixes), GEMM tiles with
and without split-K, and the fused decode GEMV (RMSNorm or SwiGLU prologue or none, with or
without the residual) up to its K limit.  Every output is held to the reference's pass rule
(2e-3 of max|ref|), and every grouped output must also equal its single-problem GEMV bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kernelforge import ops
from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu

REL_TOL = 2e-3
DEV = "cuda"
SEED = 20261202


def _draw_k(rng: np.random.Generator, g: int, kmax: int) -> int:
    special = [1024, 1536, 2048, 2112, 5632]
    if rng.random() < 0.3:
        k = int(rng.choice(special))
        if k % g == 0 and k <= kmax:
            return k
    return g * int(rng.integers(1, kmax // g + 1))


def _weight(n: int, k: int, g: int, seed: int):
    rng = np.random.Generator(np.random.PCG64(seed))
    w = rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)
    packed, scales = o.quantize_weight(w, g)
    return packed, scales, torch.from_numpy(packed).to(DEV), torch.from_numpy(scales).to(DEV)


def _random_packed(n: int, k: int, g: int, seed: int):
    """Random nibbles and scales in [1e-3, 1e-2): the kernels take any packed word, and this skips
    quantizing a float weight on the CPU."""
    rng = np.random.Generator(np.random.PCG64(seed))
    packed = rng.integers(-(2**31), 2**31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
    scales = (rng.random((n, k // g), dtype=np.float32) * 0.009 + 0.001).astype(np.float16)
    return packed, scales, torch.from_numpy(packed).to(DEV), torch.from_numpy(scales).to(DEV)


def _x(m: int, k: int, seed: int) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    return rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)


def _cases(kind: str, count: int):
    rng = np.random.Generator(np.random.PCG64(SEED + {"gemv": 0, "grouped": 1, "gemm": 2, "fused": 3}[kind]))
    out = []
    for i in range(count):
        g = int(rng.choice([64, 128]))
        if kind == "gemv":
            out.append((i, int(rng.integers(1, 9)), int(rng.integers(1, 4097)), _draw_k(rng, g, 6144), g))
        elif kind == "gemm":
            out.append((i, int(rng.integers(5, 301)), 64 * int(rng.integers(1, 33)), _draw_k(rng, g, 4096), g))
        elif kind == "fused":  # (i, N, K, G, prologue 0 none / 1 RMSNorm / 2 SwiGLU, residual)
            out.append((i, int(rng.integers(1, 6001)), _draw_k(rng, g, 10240), g, int(rng.integers(0, 3)),
                        bool(rng.random() < 0.5)))
        else:
            problems = [(int(rng.integers(1, 3001)), _draw_k(rng, g, 5632)) for _ in range(int(rng.integers(2, 9)))]
            out.append((i, int(rng.integers(1, 5)), problems, g))
    return out


def _check(error_log, suite, got: torch.Tensor, x, packed, scales, g, case, shape):
    ref = o.linear_ref_fp32(x, packed, scales, g)
    arr = got.float().cpu().numpy()
    assert got.shape == ref.shape and np.isfinite(arr).all(), case
    err = o.max_rel_err(arr, ref)
    error_log.add(suite, case=case, shape=shape, group=g, max_rel_err=err, passed=err <= REL_TOL)
    assert err <= REL_TOL, f"{case} {shape} G={g}: rel err {err:.3e}"


@pytest.mark.parametrize("i,m,n,k,g", _cases("gemv", 40))
def test_random_gemv(error_log, i, m, n, k, g):
    packed, scales, dp, ds = _weight(n, k, g, SEED + 100 + i)
    x = _x(m, k, SEED + 200 + i)
    _check(error_log, "int4_gemv", ops.int4_gemv(torch.from_numpy(x).to(DEV), dp, ds, g), x, packed, scales, g,
           f"random_gemv_{i}", [m, n, k])


@pytest.mark.parametrize("i,m,problems,g", _cases("grouped", 20))
def test_random_grouped_gemv(error_log, i, m, problems, g):
    hosts, xs, ps, ss = [], [], [], []
    for j, (n, k) in enumerate(problems):
        packed, scales, dp, ds = _weight(n, k, g, SEED + 1000 * (i + 1) + j)
        x = _x(m, k, SEED + 5000 * (i + 1) + j)
        hosts.append((x, packed, scales))
        xs.append(torch.from_numpy(x).to(DEV))
        ps.append(dp)
        ss.append(ds)
    ys = ops.int4_gemv_grouped(xs, ps, ss, g)
    for j, (n, k) in enumerate(problems):
        single = ops.int4_gemv(xs[j], ps[j], ss[j], g)
        assert torch.equal(ys[j], single), f"random_grouped_{i} problem {j} ({n} x {k}): grouped differs from single"
        x, packed, scales = hosts[j]
        _check(error_log, "int4_gemv_grouped", ys[j], x, packed, scales, g, f"random_grouped_{i}_{j}", [m, n, k])


@pytest.mark.parametrize("i,m,n,k,g", _cases("gemm", 20))
def test_random_gemm(error_log, i, m, n, k, g):
    packed, scales, dp, ds = _weight(n, k, g, SEED + 300 + i)
    x = _x(m, k, SEED + 400 + i)
    y = ops.int4_gemm(torch.from_numpy(x).to(DEV), dp, ds, g)
    _check(error_log, "int4_gemm", y, x, packed, scales, g, f"random_gemm_{i}", [m, n, k])
    # split-K and in-block k-group partials are summed in fixed order: a second call, same bits
    assert torch.equal(y, ops.int4_gemm(torch.from_numpy(x).to(DEV), dp, ds, g))


@pytest.mark.parametrize("i,n,k,g,pro,res", _cases("fused", 24))
def test_random_fused_gemv(error_log, i, n, k, g, pro, res):
    """int4_linear_fused against the oracle fed the prologue in float64 (RMSNorm: x (mean(x^2) +
    eps)^-1/2 w; SwiGLU: fp16(silu(g)) u; each rounded to fp16 as the op's input), plus the
    residual added to the fp16 product."""
    packed, scales, dp, ds = _random_packed(n, k, g, SEED + 500 + i)
    rng = np.random.Generator(np.random.PCG64(SEED + 600 + i))
    x = rng.standard_normal((1, k), dtype=np.float32).astype(np.float16)
    aux = ((rng.random(k, dtype=np.float32) + 0.5) if pro == 1 else rng.standard_normal((1, k), dtype=np.float32))
    aux = aux.astype(np.float16)
    r = (rng.standard_normal((1, n), dtype=np.float32) * 4).astype(np.float16) if res else None
    kw = {}
    if pro == 1:
        kw["norm_weight"] = torch.from_numpy(aux).to(DEV)
    elif pro == 2:
        kw["up"] = torch.from_numpy(aux).to(DEV)
    if res:
        kw["residual"] = torch.from_numpy(r).to(DEV)
    y = ops.int4_linear_fused(torch.from_numpy(x).to(DEV), dp, ds, g, **kw)
    xd = x.astype(np.float64)
    if pro == 1:
        xin = (xd / np.sqrt((xd * xd).mean() + 1e-5) * aux.astype(np.float64)).astype(np.float16)
    elif pro == 2:
        xin = ((xd / (1.0 + np.exp(-xd))).astype(np.float16).astype(np.float64) * aux.astype(np.float64)).astype(np.float16)
    else:
        xin = x
    ref = o.linear_ref_fp32(xin, packed, scales, g)
    if res:
        ref = r.astype(np.float32) + ref.astype(np.float16).astype(np.float32)
    arr = y.float().cpu().numpy()
    assert y.shape == (1, n) and np.isfinite(arr).all()
    err = o.max_rel_err(arr, ref)
    error_log.add("int4_gemv_fused", case=f"random_fused_{i}", shape=[1, n, k], group=g, max_rel_err=err,
                  passed=err <= REL_TOL)
    assert err <= REL_TOL, f"random_fused_{i} N={n} K={k} G={g} prologue={pro} residual={res}: rel err {err:.3e}"
