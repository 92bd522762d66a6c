"""The package's format producer (kernelforge.quantize, torch) against the pinned oracle.

Restates the reference's tests/test_quantize.py (KATs, invariants, rejections)
for the package, and checks that its packed bytes and scales are bit-identical
to the numpy oracle on seeded, crafted and golden inputs.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest
import torch

from kernelforge import quantize as kq
from oracle import int4_oracle as o

GOLDEN = Path(__file__).resolve().parent / "golden" / "int4_cases.npz"


def _cases():
    data = np.load(GOLDEN)
    names = sorted({k.split("__")[0] for k in data.files})
    return data, names


def test_pack_unpack_roundtrip_is_exact():
    g = torch.Generator().manual_seed(0)
    q = torch.randint(-8, 8, (64, 256), generator=g, dtype=torch.int8)
    assert torch.equal(kq.unpack_int4(kq.pack_int4(q)), q)


def test_bit_layout_matches_docstring():
    q = torch.arange(0, 8, dtype=torch.int8).reshape(1, 8)
    word = kq.pack_int4(q).item() & 0xFFFFFFFF
    assert [(word >> (4 * i)) & 0xF for i in range(8)] == [8, 10, 12, 14, 9, 11, 13, 15]
    for i in range(4):
        pair = (word >> (4 * i)) & 0x000F000F
        assert (pair & 0xF, pair >> 16) == (2 * i + 8, 2 * i + 9)


@pytest.mark.parametrize("group_size", [64, 128])
def test_quantization_error_is_bounded(group_size):
    g = torch.Generator().manual_seed(1)
    w = torch.randn(256, 1024, generator=g) * 0.02
    qw = kq.quantize_weight(w, group_size)
    w_hat = kq.dequantize(qw, torch.float32)
    step = qw.scales.float().repeat_interleave(group_size, dim=1)
    assert ((w_hat - w).abs() <= 0.5 * step + 1e-8).all()
    stats = kq.quantization_error(w, qw)
    assert stats["rel_fro_err"] < 0.15
    assert stats["bits_per_weight"] == pytest.approx(4 + 16 / group_size)


def test_quantization_error_matches_oracle_and_exact_values():
    """kernelforge.quantize.quantization_error (torch, fp32) against the oracle's (numpy, float64
    rmse) and the exact rational errors of a crafted weight; then against the oracle on a seeded
    gaussian weight (reference kernelforge/quantize.py:117-126)."""
    import math

    from exact_cases import crafted_error_case

    w, errs = crafted_error_case()
    qw = kq.quantize_weight(torch.from_numpy(w), 64)
    stats = kq.quantization_error(torch.from_numpy(w), qw)
    ref = o.quantization_error(w, qw.packed.numpy(), qw.scales.numpy(), 64)
    assert stats["max_abs_err"] == ref["max_abs_err"] == float(max(abs(e) for e in errs))
    assert stats["rmse"] == pytest.approx(math.sqrt(sum(e * e for e in errs) / len(errs)), rel=1e-6)
    assert stats["rmse"] == pytest.approx(ref["rmse"], rel=1e-6)
    assert stats["rel_fro_err"] == pytest.approx(ref["rel_fro_err"], rel=1e-6)
    assert stats["bits_per_weight"] == ref["bits_per_weight"] == 4 + 16 / 64
    g = torch.Generator().manual_seed(3)
    wg = torch.randn(96, 512, generator=g) * 0.02
    for gs in (64, 128):
        qg = kq.quantize_weight(wg, gs)
        a = kq.quantization_error(wg, qg)
        b = o.quantization_error(wg.numpy(), qg.packed.numpy(), qg.scales.numpy(), gs)
        assert a["max_abs_err"] == b["max_abs_err"]
        for key in ("rmse", "rel_fro_err"):
            assert a[key] == pytest.approx(b[key], rel=1e-5)
        assert a["bits_per_weight"] == b["bits_per_weight"]


def test_absmax_maps_to_seven_and_zero_groups_are_safe():
    w = torch.zeros(2, 128)
    w[0, 5] = -3.5
    w[0, 9] = 1.0
    q, s = kq.quantize_int4(w, 128)
    assert q[0, 5].item() == -7 and s[0, 0].item() == 0.5
    assert (q[1] == 0).all() and s[1, 0].item() == 1.0


def test_rejections():
    with pytest.raises(ValueError, match="not a multiple of group_size"):
        kq.quantize_weight(torch.randn(16, 200), 128)
    with pytest.raises(ValueError, match="group_size"):
        kq.quantize_weight(torch.randn(16, 256), 32)
    with pytest.raises(ValueError, match="2-D"):
        kq.quantize_weight(torch.randn(4, 16, 256), 128)
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        kq.pack_int4(torch.full((1, 8), 9, dtype=torch.int8))


@pytest.mark.parametrize("seed,n,k,g", [(0, 64, 256, 64), (1, 33, 512, 128), (2, 256, 2048, 128),
                                        (3, 128, 1536, 64)])
def test_package_quantizer_bit_exact_vs_oracle(seed, n, k, g):
    w, _, packed, scales = o.seeded_case(1, n, k, g, seed)
    qw = kq.quantize_weight(torch.from_numpy(w), g)
    assert np.array_equal(qw.packed.numpy(), packed)
    assert np.array_equal(qw.scales.numpy().view(np.uint16), scales.view(np.uint16))
    assert np.array_equal(kq.dequantize(qw, torch.float16).numpy().view(np.uint16),
                          o.dequantize_fp16(packed, scales, g).view(np.uint16))
    assert np.array_equal(kq.dequantize(qw, torch.float32).numpy(), o.dequantize_fp32(packed, scales, g))


def test_package_quantizer_on_golden_cases():
    data, names = _cases()
    for name in names:
        g = int(data[f"{name}__g"])
        qw = kq.quantize_weight(torch.from_numpy(data[f"{name}__w"]), g)
        assert np.array_equal(qw.packed.numpy(), data[f"{name}__packed"]), name
        assert np.array_equal(qw.scales.numpy().view(np.uint16), data[f"{name}__scales"].view(np.uint16)), name
        assert np.array_equal(kq.dequantize(qw).numpy().view(np.uint16), data[f"{name}__w_hat16"].view(np.uint16))


def test_golden_cases_match_oracle():
    """The committed fixtures still agree with the (pinned) oracle."""
    data, names = _cases()
    for name in names:
        g = int(data[f"{name}__g"])
        packed, scales = o.quantize_weight(data[f"{name}__w"], g)
        assert np.array_equal(packed, data[f"{name}__packed"])
        y = o.linear_ref_fp32(data[f"{name}__x"], packed, scales, g)
        assert np.array_equal(y, data[f"{name}__y_ref32"])


def test_quantized_weight_nbytes():
    qw = kq.quantize_weight(torch.randn(64, 256) * 0.02, 128)
    assert qw.nbytes == 64 * 32 * 4 + 64 * 2 * 2
    assert qw.shape == (64, 256) and qw.packed.dtype == torch.int32 and qw.scales.dtype == torch.float16
