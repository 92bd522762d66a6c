"""Pins the CPU oracle (oracle/) before anything is checked against it.

Each check is chosen so a plausible mistake in the oracle fails it: a wrong
nibble order, round-half-away instead of ties-to-even, a scale not rounded to
fp16, the tiny-clamp applied after the fp16 cast, a double rounding in the
fp16 dequant, a wrong LCG draw order.  The checks come from the reference's
own tests (KATs), from exact rational arithmetic, from brute force on tiny
inputs, and from the independent C restatement (oracle/kf_oracle.c).
"""

from __future__ import annotations

import json
from fractions import Fraction
from pathlib import Path

import numpy as np
import pytest

from oracle import c_oracle
from oracle import int4_oracle as o
from exact_cases import crafted_error_case

GOLDEN = Path(__file__).resolve().parent / "golden"


def _kats():
    return json.loads((GOLDEN / "reference_kats.json").read_text())


# ---------------------------------------------------------------------------
# Packing (kernelforge/quantize.py:74-97)
# ---------------------------------------------------------------------------

def test_bit_layout_kat():
    """Reference tests/test_quantize.py:16-25: q = 0..7 packs to nibbles [8,10,12,14,9,11,13,15]."""
    kat = _kats()["bit_layout"]
    q = np.array([kat["q"]], dtype=np.int8)
    word = int(o.pack_int4(q)[0, 0]) & 0xFFFFFFFF
    assert word == int(kat["word_hex"], 16)
    assert int(o.pack_int4(q)[0, 0]) == kat["word_int32"]
    assert [(word >> (4 * i)) & 0xF for i in range(8)] == kat["nibbles"]
    for i in range(4):
        pair = (word >> (4 * i)) & 0x000F000F
        assert (pair & 0xF, pair >> 16) == (2 * i + 8, 2 * i + 9)
    assert int(c_oracle.pack(q)[0, 0]) == kat["word_int32"]


@pytest.mark.parametrize("pos", range(8))
def test_every_nibble_value_at_every_position(pos):
    """Exhaustive: all 16 values of u at all 8 nibble positions, packer and unpacker."""
    koff = o.NIBBLE_K[pos]
    for u in range(16):
        q = np.zeros((1, 8), dtype=np.int8)
        q[0, koff] = u - 8
        word = int(o.pack_int4(q)[0, 0]) & 0xFFFFFFFF
        nib = [(word >> (4 * i)) & 0xF for i in range(8)]
        assert nib[pos] == u
        assert all(v == 8 for i, v in enumerate(nib) if i != pos)
        assert np.array_equal(o.unpack_int4(o.pack_int4(q)), q)
        assert np.array_equal(c_oracle.unpack(o.pack_int4(q)), q)


def test_pack_matches_c_host_packer_and_roundtrips():
    rng = np.random.default_rng(0)
    q = rng.integers(-8, 8, size=(64, 256), dtype=np.int8)
    packed = o.pack_int4(q)
    assert packed.dtype == np.int32 and packed.shape == (64, 32)
    assert np.array_equal(packed, c_oracle.pack(q))
    assert np.array_equal(o.unpack_int4(packed), q)
    assert np.array_equal(c_oracle.unpack(packed), q)


def test_pack_rejects_out_of_range_and_bad_shape():
    with pytest.raises(ValueError, match=r"\[-8, 7\]"):
        o.pack_int4(np.full((1, 8), 9, dtype=np.int8))
    with pytest.raises(ValueError, match="multiple of 8"):
        o.pack_int4(np.zeros((2, 12), dtype=np.int8))


# ---------------------------------------------------------------------------
# Quantizer (kernelforge/quantize.py:61-71)
# ---------------------------------------------------------------------------

def test_quantizer_kat_absmax_and_zero_group():
    """Reference tests/test_quantize.py:43-49."""
    kat = _kats()["quantizer"]
    w = np.zeros((2, 128), dtype=np.float32)
    for idx, val in kat["row0_nonzero"]:
        w[0, idx] = val
    q, s = o.quantize_int4(w, 128)
    assert q[0, 5] == kat["q_row0_idx5"] and q[0, 9] == kat["q_row0_idx9"]
    assert float(s[0, 0]) == kat["scale_row0"]
    assert (q[1] == 0).all() and float(s[1, 0]) == kat["scale_zero_group"]


def _fp16_nearest(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest fp16 value, ties to even (normal range only)."""
    assert v > 0
    e = v.numerator.bit_length() - v.denominator.bit_length()
    while Fraction(2) ** e > v:
        e -= 1
    while Fraction(2) ** (e + 1) <= v:
        e += 1
    e = max(e, -14)
    ulp = Fraction(2) ** (e - 10)
    lo = (v // ulp) * ulp
    hi = lo + ulp
    if v - lo < hi - v:
        return lo
    if v - lo > hi - v:
        return hi
    return lo if (lo / ulp) % 2 == 0 else hi


def _fp32_nearest(v: Fraction) -> Fraction:
    """Round an exact rational to the nearest fp32 value, ties to even (normal range)."""
    if v == 0:
        return Fraction(0)
    sign = -1 if v < 0 else 1
    a = abs(v)
    e = a.numerator.bit_length() - a.denominator.bit_length()
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    ulp = Fraction(2) ** (e - 23)
    lo = (a // ulp) * ulp
    hi = lo + ulp
    if a - lo < hi - a:
        r = lo
    elif a - lo > hi - a:
        r = hi
    else:
        r = lo if (lo / ulp) % 2 == 0 else hi
    return sign * r


def _brute_quantize_group(w: np.ndarray) -> tuple[list[int], Fraction]:
    """Exact-arithmetic restatement for one group: fp32 absmax/7, clamp to 2^-14, RNE to fp16,
    then q = the integer in [-8, 7] nearest to fl32(w / s), ties to even."""
    absmax = max(abs(Fraction(float(v))) for v in w)
    if absmax == 0:
        return [0] * len(w), Fraction(1)
    s = _fp16_nearest(max(_fp32_nearest(absmax / 7), Fraction(1, 2 ** 14)))
    qs = []
    for v in w:
        r = _fp32_nearest(Fraction(float(v)) / s)
        best = min(range(-8, 8), key=lambda c: (abs(r - c), c % 2))
        qs.append(best)
    return qs, s


@pytest.mark.parametrize("case", ["gaussian", "ties", "tiny", "mixed"])
def test_quantizer_brute_force(case):
    rng = np.random.default_rng(7)
    if case == "gaussian":
        w = (rng.standard_normal((3, 64)) * 0.02).astype(np.float32)
    elif case == "ties":
        # s = 0.5 exactly (absmax 3.5); w / s lands on exact .5 ties: 2.5 -> 2, 1.5 -> 2, -0.5 -> 0, -2.5 -> -2
        w = np.zeros((1, 64), dtype=np.float32)
        w[0, :6] = [3.5, 1.25, 0.75, -0.25, -1.25, 0.25]
    elif case == "tiny":
        # absmax / 7 is below 2^-14: the scale clamps to 2^-14 before the fp16 cast.
        w = np.full((1, 64), 1e-6, dtype=np.float32)
        w[0, 3] = -3e-6
    else:
        w = (rng.standard_normal((2, 64)) * rng.choice([1e-3, 1.0, 30.0], size=(2, 1))).astype(np.float32)
    q, s = o.quantize_int4(w, 64)
    for r in range(w.shape[0]):
        bq, bs = _brute_quantize_group(w[r])
        assert Fraction(float(s[r, 0])) == bs
        assert q[r].tolist() == bq
    if case == "ties":
        assert q[0, :6].tolist() == [7, 2, 2, 0, -2, 0]


def test_quantizer_invariants_and_error_stats():
    """Reference tests/test_quantize.py:28-40: half-step bound, rel-Frobenius < 0.15, 4 + 16/G bits."""
    rng = np.random.default_rng(1)
    w = (rng.standard_normal((256, 1024)) * 0.02).astype(np.float32)
    for g in (64, 128):
        packed, scales = o.quantize_weight(w, g)
        w_hat = o.dequantize_fp32(packed, scales, g)
        step = np.repeat(scales.astype(np.float32), g, axis=1)
        assert (np.abs(w_hat - w) <= 0.5 * step + 1e-8).all()
        stats = o.quantization_error(w, packed, scales, g)
        assert stats["rel_fro_err"] < 0.15
        assert stats["bits_per_weight"] == pytest.approx(4 + 16 / g)


def test_quantization_error_exact_on_crafted_weight():
    """max_abs_err, rmse, rel_fro_err and bits_per_weight against exact rational values."""
    import math

    w, errs = crafted_error_case()
    packed, scales = o.quantize_weight(w, 64)
    stats = o.quantization_error(w, packed, scales, 64)
    max_abs = max(abs(e) for e in errs)
    assert max_abs == 1 and min(errs) == -max_abs  # the largest error is negative
    mean_sq = sum(e * e for e in errs) / len(errs)
    w_sq = sum(Fraction(float(v)) ** 2 for v in w.ravel())
    assert stats["max_abs_err"] == float(max_abs)
    assert stats["rmse"] == pytest.approx(math.sqrt(mean_sq), rel=1e-12)
    assert stats["rel_fro_err"] == pytest.approx(math.sqrt(sum(e * e for e in errs) / w_sq), rel=1e-6)
    assert stats["bits_per_weight"] == 8.0 * (packed.size * 4 + scales.size * 2) / w.size == 4 + 16 / 64
    # rmse is a root of a mean: neither the mean square nor the root of the sum
    assert abs(stats["rmse"] - float(mean_sq)) > 1e-3
    assert abs(stats["rmse"] - math.sqrt(sum(e * e for e in errs))) > 1e-3


def test_quantizer_rejections():
    with pytest.raises(ValueError, match="not a multiple of group_size"):
        o.quantize_weight(np.zeros((16, 200), dtype=np.float32), 128)
    with pytest.raises(ValueError, match="group_size"):
        o.quantize_weight(np.zeros((16, 256), dtype=np.float32), 32)
    with pytest.raises(ValueError, match="2-D"):
        o.quantize_weight(np.zeros((4, 16, 256), dtype=np.float32), 128)


# ---------------------------------------------------------------------------
# fp16 conversion and dequantization (kernelforge/quantize.py:108-114)
# ---------------------------------------------------------------------------

def test_c_fp16_conversion_matches_ieee_on_all_halfway_points():
    """The C oracle's float->half RNE against numpy on every fp16 value, its neighbours and the exact ties."""
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16)  # all finite non-negative fp16
    f = h.astype(np.float32)
    nxt = np.nextafter(h, np.float16(np.inf)).astype(np.float32)
    mid = ((f.astype(np.float64) + nxt.astype(np.float64)) / 2).astype(np.float32)  # exact ties
    sample = np.concatenate([f, -f, mid, -mid, np.nextafter(mid, np.float32(0)), np.nextafter(mid, np.float32(1e9)),
                             np.array([1e-9, 65504.0, 65519.0, 65520.0, 1e6], dtype=np.float32)])
    sample = sample[::7]  # ~40k values keep the ctypes loop to a few seconds
    got = c_oracle.f32_to_f16_bits(sample)
    want = sample.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)


def test_dequant_fp16_single_rounding_exact():
    """fp16(q * s) for every q and a spread of scales equals the exactly-rounded rational product."""
    rng = np.random.default_rng(3)
    scales = np.concatenate([rng.uniform(1e-4, 0.05, 40), [2 ** -14, 0.5, 1.0, 0.000977, 3.3e-3]]).astype(np.float16)
    n = len(scales)
    q = np.tile(np.arange(-8, 8, dtype=np.int8), (n, 4))  # K = 64, every q value 4 times
    packed = o.pack_int4(q)
    w16 = o.dequantize_fp16(packed, scales.reshape(n, 1), 64)
    assert np.array_equal(w16.view(np.uint16), c_oracle.dequant_fp16(packed, scales.reshape(n, 1), 64).view(np.uint16))
    for r in range(n):
        for c in range(16):
            exact = Fraction(int(q[r, c])) * Fraction(float(scales[r]))
            want = 0.0 if exact == 0 else float(np.sign(float(exact))) * float(_fp16_nearest(abs(exact)))
            assert float(w16[r, c]) == want


def test_dequant_fp32_is_exact():
    rng = np.random.default_rng(4)
    w = (rng.standard_normal((32, 256)) * 0.02).astype(np.float32)
    packed, scales = o.quantize_weight(w, 128)
    exact = o.unpack_int4(packed).astype(np.float64) * np.repeat(scales.astype(np.float64), 128, axis=1)
    assert np.array_equal(o.dequantize_fp32(packed, scales, 128).astype(np.float64), exact)


# ---------------------------------------------------------------------------
# FP32 / f64 references (tests/test_gemm.py:27-45, sanitize_gemm.cu:58-66)
# ---------------------------------------------------------------------------

def test_linear_refs_against_brute_force_loop():
    rng = np.random.default_rng(5)
    m, n, k, g = 3, 5, 128, 64
    w = (rng.standard_normal((n, k)) * 0.02).astype(np.float32)
    x = rng.standard_normal((m, k)).astype(np.float16)
    packed, scales = o.quantize_weight(w, g)
    q = o.unpack_int4(packed)
    brute = np.zeros((m, n))
    for i in range(m):
        for j in range(n):
            brute[i, j] = sum(float(x[i, kk]) * int(q[j, kk]) * float(scales[j, kk // g]) for kk in range(k))
    assert np.allclose(o.linear_ref_f64(x, packed, scales, g), brute, rtol=1e-12, atol=1e-12)
    assert np.allclose(c_oracle.ref_f64(x, packed, scales, g), brute, rtol=1e-12, atol=1e-12)
    assert o.max_rel_err(o.linear_ref_fp32(x, packed, scales, g), brute) < 1e-5


# The pass rule every GPU parity assertion goes through (tests/test_gemm.py:36-45: err <= 2e-3 *
# scale, err = max|out - ref|, scale = max|ref|, both over the whole tensor).  Every value is a
# dyadic rational, exact in fp16 and float64, so each expected ratio is exact.  In the first case
# the largest error is negative and sits at another element than the largest |ref|, which is
# negative too; the wrong readings each give another number:
#   per-element |e|/|ref| -> 1.0; mean |e| -> 0.1042; max(out - ref) without abs -> 0.125;
#   scale from out -> 0.1786; max(ref) without abs -> 0.3125; rms of e -> 0.1169.
# The second case puts the error and the largest |ref| in different rows and columns (a
# per-row or per-column scale gives 1.0).
_NAN = object()
MAX_REL_ERR_CASES = [
    ("negatives_apart", [0.25, 1.375, -3.5], [0.125, 2.0, -4.0], 0.15625),
    ("two_d_whole_tensor", [[1.0, 0.25], [0.25, -8.0]], [[0.5, 0.25], [0.25, -8.0]], 0.0625),
    ("exact", [[-1.5, 0.75]], [[-1.5, 0.75]], 0.0),
    ("nan_beside_exact", [np.nan, 1.0], [1.0, 1.0], _NAN),      # fmax would drop the NaN: 0.0
    ("nan_beside_error", [0.5, np.nan, 2.0], [0.5, 1.0, 1.0], _NAN),
    ("inf_out", [np.inf, 1.0], [1.0, 1.0], float("inf")),
    ("zero_ref_exact", [0.0, -0.0, 0.0], [0.0, 0.0, 0.0], 0.0),
    ("zero_ref_tiny_error", [0.0, 2.0 ** -24], [0.0, 0.0], float("inf")),  # the reference fails it
]


@pytest.mark.parametrize("name,out,ref,want", MAX_REL_ERR_CASES, ids=[c[0] for c in MAX_REL_ERR_CASES])
def test_max_rel_err_hand_computed(name, out, ref, want):
    """oracle.max_rel_err and the native check's kfo_max_rel_err_f16 on hand-computed cases, and
    the pass decision (<= 2e-3) equal to the reference's err <= 2e-3 * scale."""
    out64 = np.array(out, dtype=np.float64)
    ref64 = np.array(ref, dtype=np.float64)
    got_np = o.max_rel_err(out64, ref64)
    got_c = c_oracle.max_rel_err_f16(out64.astype(np.float16), ref64)
    for got in (got_np, got_c):
        if want is _NAN:
            assert np.isnan(got), name
        else:
            assert got == want, (name, got)
    with np.errstate(invalid="ignore"):
        err = np.max(np.abs(out64 - ref64))
        ref_pass = bool(err <= 2e-3 * np.max(np.abs(ref64)))
    assert (got_np <= 2e-3) == ref_pass == (got_c <= 2e-3), name


def test_max_rel_err_refuses_shape_mismatch_and_empty_is_zero():
    """A transposed or flattened out must not broadcast against ref into an N x N difference."""
    with pytest.raises(ValueError, match="shape"):
        o.max_rel_err(np.zeros((1, 3)), np.zeros((3, 1)))
    with pytest.raises(ValueError, match="shape"):
        o.max_rel_err(np.zeros(3), np.zeros((1, 3)))
    assert o.max_rel_err(np.zeros((0, 4)), np.zeros((0, 4))) == 0.0
    assert c_oracle.max_rel_err_f16(np.zeros(0, np.float16), np.zeros(0)) == 0.0


def test_max_rel_err_on_a_gemv_sized_output():
    """A seeded [1, 5632] output: one element off by exactly 2e-3 * max|ref| (+/- a little) decides
    pass / fail at the reference's boundary, in both implementations."""
    rng = np.random.default_rng(11)
    ref = rng.standard_normal((1, 5632))
    out16 = ref.astype(np.float16)
    base = o.max_rel_err(out16.astype(np.float64), ref)
    assert base < 2.0 ** -11 and c_oracle.max_rel_err_f16(out16, ref) == base
    scale = np.abs(ref).max()
    j = int(np.argmin(np.abs(ref)))  # far from the largest |ref|
    for factor, passes in ((0.9, True), (1.1, False)):
        bad = ref.copy()
        bad[0, j] += factor * 2e-3 * scale
        bad16 = bad.astype(np.float16)
        assert (o.max_rel_err(bad16.astype(np.float64), ref) <= 2e-3) is passes
        assert (c_oracle.max_rel_err_f16(bad16, ref) <= 2e-3) is passes


def test_linear_ref_is_linear_in_x():
    rng = np.random.default_rng(6)
    w = (rng.standard_normal((64, 256)) * 0.02).astype(np.float32)
    packed, scales = o.quantize_weight(w, 128)
    x1 = rng.standard_normal((2, 256)).astype(np.float16)
    x2 = rng.standard_normal((2, 256)).astype(np.float16)
    y1 = o.linear_ref_f64(x1, packed, scales, 128)
    y2 = o.linear_ref_f64(x2, packed, scales, 128)
    y12 = o.linear_ref_f64(np.concatenate([x1, x2]), packed, scales, 128)
    assert np.allclose(y12, np.concatenate([y1, y2]))
    xs = (x1.astype(np.float64) + x2.astype(np.float64))
    w_hat = o.dequantize_fp32(packed, scales, 128).astype(np.float64)
    assert np.allclose(xs @ w_hat.T, y1 + y2)


# ---------------------------------------------------------------------------
# The reference's torch-free workload (sanitize_gemm.cu:21-66)
# ---------------------------------------------------------------------------

@pytest.mark.parametrize("group", [64, 128])
def test_lcg_workload_numpy_matches_c(group):
    q, s, p, xs = o.lcg_workload(group)
    cq, cs, cp, cxs = c_oracle.lcg_workload(group)
    assert np.array_equal(q, cq)
    assert np.array_equal(s.view(np.uint16), cs.view(np.uint16))
    assert np.array_equal(p, cp)
    for m in xs:
        assert np.array_equal(xs[m].view(np.uint16), cxs[m].view(np.uint16))
    assert q.min() == -8 and q.max() == 7
    assert 0.01 <= float(s.astype(np.float32).min()) and float(s.astype(np.float32).max()) <= 0.0301


@pytest.mark.parametrize("group", [64, 128])
def test_lcg_workload_digest(group):
    """SHA-256 of the workload bytes, committed so any machine can confirm it regenerates the same inputs."""
    import hashlib

    q, s, p, xs = o.lcg_workload(group)
    h = hashlib.sha256()
    for a in (p, s.view(np.uint16), *[xs[m].view(np.uint16) for m in sorted(xs)]):
        h.update(np.ascontiguousarray(a).tobytes())
    assert h.hexdigest() == _kats()["lcg_sha256"][str(group)]


def test_algorithmic_bytes_formula():
    """BASELINE totals: TinyLlama 7 linears at M=1 move 22,779,904 B; Qwen2.5 24,209,920 B."""
    kat = _kats()["bytes"]
    tl = [(2048, 2048), (256, 2048), (256, 2048), (2048, 2048), (5632, 2048), (5632, 2048), (2048, 5632)]
    qw = [(1536, 1536), (256, 1536), (256, 1536), (1536, 1536), (8960, 1536), (8960, 1536), (1536, 8960)]
    assert sum(o.algorithmic_bytes(1, n, k, 128) for n, k in tl) == kat["tinyllama_7"]
    assert sum(o.algorithmic_bytes(1, n, k, 128) for n, k in qw) == kat["qwen_7"]
    assert o.gemm_flops(2048, 5632, 2048) == kat["gate_m2048_flops"]


@pytest.mark.parametrize("n,k,g", [(1, 128, 128), (16, 256, 64), (37, 384, 128), (40, 256, 64)])
def test_reorder_mfma16_by_definition(n, k, g):
    """The layout of kf_int4_reorder_mfma16 element by element, as the header states it."""
    rng = np.random.default_rng(n * 7 + k)
    packed = rng.integers(-2**31, 2**31, size=(n, k // 8), dtype=np.int64).astype(np.int32)
    scales = rng.standard_normal((n, k // g)).astype(np.float16)
    pr, sr = o.reorder_mfma16(packed, scales, g)
    nb, nss = -(-n // 16), k // 128
    assert pr.shape == (nb * 16 * k // 8,) and sr.shape == (nb * 16 * k // g,)
    piece = 0
    for b in range(nb):
        for s in range(nss):
            for lane in range(64):
                row = min(16 * b + lane % 16, n - 1)
                w0 = 16 * s + 4 * (lane // 16)
                assert np.array_equal(pr[4 * piece:4 * piece + 4], packed[row, w0:w0 + 4])
                piece += 1
    i = 0
    for b in range(nb):
        for j in range(k // g):
            for c in range(16):
                assert sr[i].view(np.uint16) == scales[min(16 * b + c, n - 1), j].view(np.uint16)
                i += 1


def test_reorder_mfma16_is_a_permutation():
    """Every 4-word piece of the source appears; padding only repeats row N-1."""
    n, k = 21, 512
    packed = np.arange(n * k // 8, dtype=np.int32).reshape(n, k // 8)  # every word distinct
    scales = np.arange(n * k // 128, dtype=np.float16).reshape(n, k // 128)
    pr, _ = o.reorder_mfma16(packed, scales, 128)
    pieces = pr.reshape(-1, 4)
    assert (pieces[:, 1:] == pieces[:, :1] + np.arange(1, 4)).all()  # pieces are whole aligned runs
    assert set(pieces[:, 0] // 4) == set(range(n * k // 32))          # every source piece present
    counts = np.bincount(pieces[:, 0] // 4 // (k // 32))
    assert (counts[:-1] == k // 32).all() and counts[-1] == (32 - n + 1) * (k // 32)  # rows 21..31 repeat row 20
    with pytest.raises(ValueError):
        o.reorder_mfma16(packed[:, :12], scales[:, :1], 128)  # K = 96


# ---------------------------------------------------------------------------
# The torch restatement timed as bench.py's CPU baseline (oracle/cpu_baseline.py)
# ---------------------------------------------------------------------------

def test_cpu_baseline_matches_numpy_oracle():
    """Unpack and fp32 dequant bit-exact against the pinned numpy oracle (every nibble value at
    every position, plus a seeded weight); the matmul within fp32 summation-order tolerance."""
    import torch

    from oracle import cpu_baseline as cb

    q = np.array([[u - 8 for u in range(16)] * 8], dtype=np.int8).reshape(16, 8)
    q = np.concatenate([np.roll(q, s, axis=1) for s in range(8)], axis=0)  # every value at every k offset
    packed = o.pack_int4(q)
    assert np.array_equal(cb.unpack_int4(torch.from_numpy(packed)).numpy(), q)
    _, x, packed, scales = o.seeded_case(3, 200, 1024, 128, seed=5)
    tp, ts = torch.from_numpy(packed), torch.from_numpy(scales)
    assert np.array_equal(cb.dequantize_fp32(tp, ts, 128).numpy(), o.dequantize_fp32(packed, scales, 128))
    y = cb.linear_fp32(torch.from_numpy(x), tp, ts, 128).numpy()
    assert o.max_rel_err(y, o.linear_ref_f64(x, packed, scales, 128)) < 1e-5
    w_hat = cb.dequantize_fp32(tp, ts, 128)
    assert np.array_equal(cb.matmul_only(torch.from_numpy(x), w_hat).numpy(), y)
