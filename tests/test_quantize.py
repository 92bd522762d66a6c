"""The package's format producer (kernelforge.quantize, torch) against the pinned oracle.

The reference's quantizer checks (tests/test_quantize.py:9-66: layout KAT, quantizer KAT,
error invariants, rejections) are data in tests/golden/reference_kats.json; the tests below
read them from there.  The packed bytes and scales are also checked bit for bit against the
numpy oracle on seeded, crafted and golden inputs.
"""

from __future__ import annotations

import json
from pathlib import Path

import numpy as np
import pytest
import torch

from kernelforge import quantize as kq
from oracle import int4_oracle as o

GOLDEN = Path(__file__).resolve().parent / "golden" / "int4_cases.npz"
KATS = json.loads((Path(__file__).resolve().parent / "golden" / "reference_kats.json").read_text())


def _cases():
    data = np.load(GOLDEN)
    names = sorted({k.split("__")[0] for k in data.files})
    return data, names


def _nibbles(word: int) -> list[int]:
    return [(word >> (4 * i)) & 0xF for i in range(8)]


def test_layout_kat_from_fixture():
    """pack_int4 of the fixture's q gives its word and nibble order; the (k 2i, k 2i+1) pairs a
    kernel reads with one mask sit in the two 16-bit halves; unpack_int4 inverts it."""
    kat = KATS["bit_layout"]
    q = torch.tensor([kat["q"]], dtype=torch.int8)
    packed = kq.pack_int4(q)
    assert packed.dtype == torch.int32 and packed.shape == (1, 1)
    assert packed.item() == kat["word_int32"]
    word = packed.item() & 0xFFFFFFFF
    assert word == int(kat["word_hex"], 16) and _nibbles(word) == kat["nibbles"]
    halves = [((word >> (4 * i)) & 0xF, (word >> (4 * i + 16)) & 0xF) for i in range(4)]
    assert halves == [(kat["q"][2 * i] + 8, kat["q"][2 * i + 1] + 8) for i in range(4)]
    assert torch.equal(kq.unpack_int4(packed), q)


@pytest.mark.parametrize("pos", range(8))
def test_every_value_at_every_nibble_round_trips(pos):
    """Exhaustive over the 16 values at each of the 8 positions of a word, against the oracle's
    packer, with every other k at q = 0 (nibble 8)."""
    koff = o.NIBBLE_K[pos]
    q = torch.zeros(16, 8, dtype=torch.int8)
    q[:, koff] = torch.arange(-8, 8, dtype=torch.int8)
    packed = kq.pack_int4(q)
    assert np.array_equal(packed.numpy(), o.pack_int4(q.numpy()))
    for u in range(16):
        nib = _nibbles(int(packed[u, 0]) & 0xFFFFFFFF)
        assert nib[pos] == u and all(v == 8 for i, v in enumerate(nib) if i != pos)
    assert torch.equal(kq.unpack_int4(packed), q)


def test_quantizer_kat_from_fixture():
    """Row 0 holds only the fixture's nonzero entries, row 1 is all zeros (one group of 128 each)."""
    kat = KATS["quantizer"]
    w = torch.zeros(2, 128)
    for idx, val in kat["row0_nonzero"]:
        w[0, idx] = val
    q, s = kq.quantize_int4(w, 128)
    assert s.dtype == torch.float16 and s.shape == (2, 1)
    assert int(q[0, 5]) == kat["q_row0_idx5"] and int(q[0, 9]) == kat["q_row0_idx9"]
    assert float(s[0, 0]) == kat["scale_row0"] and float(s[1, 0]) == kat["scale_zero_group"]
    others = [i for i in range(128) if i not in {idx for idx, _ in kat["row0_nonzero"]}]
    assert not q[0, others].any() and not q[1].any()


@pytest.mark.parametrize("group", KATS["invariants"]["groups"])
def test_error_invariants_from_fixture(group):
    """The fixture's bounds on a seeded weight of its shape: every element within the stated
    fraction of its group's step (in float64; one part in 2^20 for the fp32 division), the
    relative Frobenius error below its bound, the stated bits per weight."""
    inv = KATS["invariants"]
    shape = (inv["weight"]["rows"], inv["weight"]["cols"])
    w = torch.randn(*shape, generator=torch.Generator().manual_seed(100 + group)) * inv["weight"]["std"]
    qw = kq.quantize_weight(w, group)
    err = (kq.dequantize(qw, torch.float32).double() - w.double()).abs()
    step = qw.scales.double().repeat_interleave(group, dim=1)
    assert bool((err <= inv["max_err_in_steps"] * step * (1 + 2.0 ** -20)).all())
    stats = kq.quantization_error(w, qw)
    assert stats["rel_fro_err"] < inv["rel_fro_err_below"]
    assert stats["bits_per_weight"] == inv["bits_per_weight"][str(group)]


@pytest.mark.parametrize("case", KATS["rejections"]["cases"], ids=lambda c: f"{c['call']}-{c['match']}")
def test_rejections_from_fixture(case):
    err = {"ValueError": ValueError, "TypeError": TypeError}[case["error"]]
    with pytest.raises(err, match=case["match"]):
        if case["call"] == "quantize_weight":
            kq.quantize_weight(torch.zeros(case["shape"]), case["group"])
        else:
            kq.pack_int4(torch.full(case["shape"], case["fill"], dtype=torch.int8))


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
