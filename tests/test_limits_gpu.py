"""The C ABI's size limits, exercised at their edges on the GPU (needs an MI355X).

* N = KF_MAX_ROWS (2^25 - 64) rows: the GEMV's largest grid (one wavefront per two rows), the
  skinny and the tiled GEMM across 2^19 column tiles, and the on-device quantizer over 2^28
  words;
* a grouped GEMV launch whose two problems add up to exactly KF_MAX_ROWS rows;
* long K: rows of 2^20 and 2^24 weights (512 KiB and 8 MiB of packed words per row), past every
  LDS copy of x, and a GEMM whose split-K partials cover K = 2^20.

Output rows are independent of each other (y[m, n] reads only x[m] and row n of the weight), so
each case checks a sample of rows against the oracle fed only those rows: the first and last
1,024 and 2,048 drawn from a fixed seed.  The whole output must be finite.  Packed words and
scales are drawn on the device (random nibbles, scales in [1e-3, 1e-2)), so no CPU quantizer
pass over gigabytes is needed; the quantizer's own case draws its weight on the device and
checks the sampled rows bit for bit.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch

from kernelforge import ops
from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu

DEV = "cuda"
REL_TOL = 2e-3
MAX_ROWS = (1 << 25) - 64  # KF_MAX_ROWS in include/kf_int4.h


def _gen(seed: int) -> torch.Generator:
    return torch.Generator(device=DEV).manual_seed(seed)


def _weight(n: int, k: int, g: int, seed: int):
    gen = _gen(seed)
    packed = torch.randint(-(2**31), 2**31 - 1, (n, k // 8), dtype=torch.int32, device=DEV, generator=gen)
    scales = (torch.rand(n, k // g, device=DEV, generator=gen) * 0.009 + 0.001).half()
    return packed, scales


def _x(m: int, k: int, seed: int) -> torch.Tensor:
    return torch.randn(m, k, device=DEV, generator=_gen(seed)).half()


def _sample(n: int, seed: int, edge: int = 1024, inner: int = 2048) -> np.ndarray:
    rng = np.random.Generator(np.random.PCG64(seed))
    idx = np.concatenate([np.arange(min(edge, n)), np.arange(max(0, n - edge), n), rng.integers(0, n, inner)])
    return np.unique(idx)


def _check_rows(error_log, suite, case, y, x, packed, scales, g, rows, xrows=None):
    """y[:, rows] (y[xrows][:, rows] for the GEMM) against the oracle on those weight rows."""
    assert torch.isfinite(y).all(), f"{case}: non-finite output"
    r = torch.from_numpy(rows).to(DEV)
    xs = x if xrows is None else x[torch.from_numpy(xrows).to(DEV)]
    got = (y if xrows is None else y[torch.from_numpy(xrows).to(DEV)])[:, r].float().cpu().numpy()
    ref = o.linear_ref_fp32(xs.cpu().numpy(), packed[r].cpu().numpy(), scales[r].cpu().numpy(), g)
    err = o.max_rel_err(got, ref)
    error_log.add(suite, case=case, shape=[int(x.shape[0]), int(packed.shape[0]), int(x.shape[1])], group=g,
                  max_rel_err=err, passed=err <= REL_TOL)
    assert err <= REL_TOL, f"{case}: rel err {err:.3e} over {rows.size} sampled rows"


@pytest.mark.parametrize("m,n,k,g", [(1, MAX_ROWS, 64, 64), (8, MAX_ROWS, 64, 64), (2, MAX_ROWS, 128, 128),
                                     (1, 64, 1 << 20, 128), (8, 64, 1 << 20, 128), (1, 3, 1 << 24, 128),
                                     (5, 3, 1 << 24, 64)])
def test_gemv_at_the_limits(error_log, m, n, k, g):
    packed, scales = _weight(n, k, g, 11 + m)
    x = _x(m, k, 12 + m)
    y = ops.int4_gemv(x, packed, scales, g)
    _check_rows(error_log, "int4_gemv", f"limit_gemv_m{m}_n{n}_k{k}", y, x, packed, scales, g, _sample(n, 13 + m))


@pytest.mark.parametrize("m", [1, 4])
def test_grouped_gemv_fills_the_row_limit(error_log, m):
    """Two problems of KF_MAX_ROWS / 2 rows each: the launch's row total is exactly the limit."""
    half = MAX_ROWS // 2
    ws = [_weight(half, 64, 64, 21), _weight(half, 128, 64, 22)]
    xs = [_x(m, 64, 23), _x(m, 128, 24)]
    ys = ops.int4_gemv_grouped(xs, [w[0] for w in ws], [w[1] for w in ws], 64)
    for j, ((packed, scales), x, y) in enumerate(zip(ws, xs, ys)):
        _check_rows(error_log, "int4_gemv_grouped", f"limit_grouped_m{m}_{j}", y, x, packed, scales, 64,
                    _sample(half, 25 + j))


@pytest.mark.parametrize("m,n,k,g", [(16, MAX_ROWS, 128, 128), (64, MAX_ROWS, 64, 64), (64, 64, 1 << 20, 128),
                                     (4096, 64, 1 << 18, 128)])
def test_gemm_at_the_limits(error_log, m, n, k, g):
    packed, scales = _weight(n, k, g, 31 + m)
    x = _x(m, k, 32 + m)
    y = ops.int4_gemm(x, packed, scales, g)
    xrows = _sample(m, 33, edge=8, inner=16) if m > 64 else None
    _check_rows(error_log, "int4_gemm", f"limit_gemm_m{m}_n{n}_k{k}", y, x, packed, scales, g, _sample(n, 34 + m),
                xrows)


def test_quantize_at_the_row_limit():
    """kf_int4_quantize over KF_MAX_ROWS x 64 fp32 weights (8 GiB), sampled rows bit for bit."""
    w = torch.randn(MAX_ROWS, 64, device=DEV, generator=_gen(41)) * 0.02
    packed, scales = ops.int4_quantize(w, 64)
    rows = torch.from_numpy(_sample(MAX_ROWS, 42)).to(DEV)
    ref_p, ref_s = o.quantize_weight(w[rows].cpu().numpy(), 64)
    assert np.array_equal(packed[rows].cpu().numpy(), ref_p)
    assert np.array_equal(scales[rows].cpu().numpy().view(np.uint16), ref_s.view(np.uint16))
