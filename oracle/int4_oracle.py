"""CPU oracle for the INT4 weight-only linear path.  TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of
``bench.py`` may import this module, and only as the checker.  The product
(``kernel-forge_amd/kernelforge``) never calls it; the GPU path fails loudly
when its HIP library is missing instead of falling back to anything here.

Everything is plain numpy restated from the reference's closed forms:

==========================  ===============================================
function                    reference it restates
==========================  ===============================================
quantize_int4               kernelforge/quantize.py:61-71
pack_int4                   kernelforge/quantize.py:74-85 (layout :12-24)
unpack_int4                 kernelforge/quantize.py:88-97
quantize_weight             kernelforge/quantize.py:100-105
dequantize_fp16 / _fp32     kernelforge/quantize.py:108-114
quantization_error          kernelforge/quantize.py:117-126
linear_ref_fp32             tests/test_gemm.py:27-33 (x.float() @ W_hat^T)
linear_ref_f64              csrc/micro/sanitize_gemm.cu:58-66
lcg_workload                csrc/micro/sanitize_gemm.cu:21-50
max_rel_err                 tests/test_gemm.py:36-45
algorithmic_bytes / flops   bench/bench_gemm.py:80,98; bench_utils.py:209-210
reorder_mfma16              no reference function: the layout contract of
                            kf_int4_reorder_mfma16 (include/kf_int4.h), the
                            weight copy the reference names as its next step
                            (docs/phase4-notes.md:59)
==========================  ===============================================

How each function is pinned (tests/test_oracle.py):

* pack/unpack: the reference's bit-layout KAT (word 0xFDB9ECA8,
  tests/test_quantize.py:16-25), an exhaustive check of all 16 nibble values
  at all 8 positions, exact round trips, and agreement with the independent C
  restatement of the reference's host packer (oracle/kf_oracle.c, after
  sanitize_gemm.cu:44-47).
* quantize_int4: the reference KATs (absmax -> +-7, all-zero group -> scale 1,
  test_quantize.py:43-49), the half-step bound and rel-Frobenius < 0.15
  (test_quantize.py:28-40), brute force (q is the nearest representable
  integer of fl32(w/s), ties to even, checked against Python's exact
  Fraction arithmetic on small inputs) and crafted tie / tiny / zero groups.
* dequantize_fp16: bit-exact against an exact-rational round-to-nearest-even
  to fp16 computed in pure Python over every (q, s) pair of a sample of
  scales; dequantize_fp32 is exact (checked against float64).
* linear_ref_fp32 / linear_ref_f64: against each other and against a brute
  force triple loop on tiny shapes, plus linearity in x.
* quantization_error: on a crafted weight whose per-element errors are exact
  rationals (tests/exact_cases.py): max_abs_err exactly, rmse and rel_fro_err
  against the exact values' square roots (a missing sqrt, a sum for a mean or
  a max without abs fails), bits_per_weight = 4 + 16/G.
* lcg_workload: against the C restatement bit for bit.
* reorder_mfma16: against a per-element loop that follows the header's wording
  (lane l of block (b, s): row 16b + l%16, words 16s + 4(l/16) .. +3), and as a
  permutation (every piece of the source appears, the padded rows repeat row
  N-1); on the GPU, the GEMM reading the copy equals the GEMM reading the
  public layout bit for bit.
"""

from __future__ import annotations

import numpy as np

SUPPORTED_GROUP_SIZES = (64, 128)
NIBBLE_K = (0, 2, 4, 6, 1, 3, 5, 7)  # k offset held at nibble position p
FP16_TINY = np.float32(2.0 ** -14)


def _check(weight: np.ndarray, group_size: int) -> tuple[int, int]:
    """Validation of kernelforge/quantize.py:50-58 (messages kept)."""
    if weight.ndim != 2:
        raise ValueError(f"weight must be 2-D [N, K], got shape {tuple(weight.shape)}")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError(f"group_size must be one of {SUPPORTED_GROUP_SIZES}, got {group_size}")
    n, k = weight.shape
    if k % group_size:
        raise ValueError(f"K={k} is not a multiple of group_size={group_size}")
    return n, k


def quantize_int4(weight: np.ndarray, group_size: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """kernelforge/quantize.py:61-71.

    scale = fp32(fp16(max(absmax / 7, 2^-14))), 1 for an all-zero group;
    q = clamp(rint(fl32(w / scale)), -8, 7) with ties to even.
    """
    n, k = _check(weight, group_size)
    w = np.asarray(weight, dtype=np.float32).reshape(n, k // group_size, group_size)
    absmax = np.abs(w).max(axis=2, keepdims=True)
    scale = np.maximum(absmax / np.float32(7.0), FP16_TINY).astype(np.float16).astype(np.float32)
    scale = np.where(absmax == 0, np.float32(1.0), scale)
    q = np.clip(np.rint(w / scale), -8, 7).astype(np.int8)
    return q.reshape(n, k), scale.reshape(n, k // group_size).astype(np.float16)


def pack_int4(q: np.ndarray) -> np.ndarray:
    """kernelforge/quantize.py:74-85: int8 [N, K] -> int32 [N, K/8]."""
    if q.ndim != 2 or q.shape[1] % 8:
        raise ValueError(f"q must be [N, K] with K a multiple of 8, got {tuple(q.shape)}")
    if q.min(initial=0) < -8 or q.max(initial=0) > 7:
        raise ValueError("q values must lie in [-8, 7]")
    n, k = q.shape
    u = (q.astype(np.uint32) + 8) & 0xF
    u = u.reshape(n, k // 8, 8)
    word = np.zeros((n, k // 8), dtype=np.uint32)
    for pos, koff in enumerate(NIBBLE_K):
        word |= u[:, :, koff] << np.uint32(4 * pos)
    return word.view(np.int32)


def unpack_int4(packed: np.ndarray) -> np.ndarray:
    """kernelforge/quantize.py:88-97: int32 [N, K/8] -> int8 [N, K]."""
    n, kw = packed.shape
    w = np.ascontiguousarray(packed).view(np.uint32)
    out = np.empty((n, kw, 8), dtype=np.int8)
    for pos, koff in enumerate(NIBBLE_K):
        out[:, :, koff] = ((w >> np.uint32(4 * pos)) & 0xF).astype(np.int8) - 8
    return out.reshape(n, kw * 8)


def quantize_weight(weight: np.ndarray, group_size: int = 128) -> tuple[np.ndarray, np.ndarray]:
    """kernelforge/quantize.py:100-105: returns (packed int32 [N, K/8], scales fp16 [N, K/G])."""
    _check(weight, group_size)
    q, scales = quantize_int4(weight, group_size)
    return pack_int4(q), scales


def dequantize_fp16(packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """kernelforge/quantize.py:112-113: fp16(q * s), one round-to-nearest-even."""
    q = unpack_int4(packed)
    n, k = q.shape
    # The product of a 4-bit integer and an 11-bit significand is exact in
    # fp32, so rounding that fp32 product to fp16 is the single RNE rounding.
    prod = q.reshape(n, k // group_size, group_size).astype(np.float32) * \
        scales.astype(np.float32)[:, :, None]
    return prod.astype(np.float16).reshape(n, k)


def dequantize_fp32(packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """kernelforge/quantize.py:114: q * s in fp32 (exact)."""
    q = unpack_int4(packed)
    n, k = q.shape
    prod = q.reshape(n, k // group_size, group_size).astype(np.float32) * \
        scales.astype(np.float32)[:, :, None]
    return prod.reshape(n, k)


def quantization_error(weight: np.ndarray, packed: np.ndarray, scales: np.ndarray, group_size: int) -> dict:
    """kernelforge/quantize.py:117-126."""
    w = np.asarray(weight, dtype=np.float32)
    err = dequantize_fp32(packed, scales, group_size) - w
    nbytes = packed.size * 4 + scales.size * 2
    return {
        "max_abs_err": float(np.abs(err).max()),
        "rmse": float(np.sqrt(np.mean(err.astype(np.float64) ** 2))),
        "rel_fro_err": float(np.linalg.norm(err) / max(np.linalg.norm(w), 1e-30)),
        "bits_per_weight": 8.0 * nbytes / w.size,
    }


def linear_ref_fp32(x16: np.ndarray, packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """tests/test_gemm.py:32: ref = x.float() @ dequantize(qw, float32).T (fp32 result)."""
    w_hat = dequantize_fp32(packed, scales, group_size)
    return np.asarray(x16, dtype=np.float32) @ w_hat.T


def linear_ref_f64(x16: np.ndarray, packed: np.ndarray, scales: np.ndarray, group_size: int) -> np.ndarray:
    """csrc/micro/sanitize_gemm.cu:58-66: double-precision sum of x * q * s."""
    w_hat = dequantize_fp32(packed, scales, group_size).astype(np.float64)
    return np.asarray(x16, dtype=np.float64) @ w_hat.T


def max_rel_err(out: np.ndarray, ref: np.ndarray) -> float:
    """tests/test_gemm.py:39-42: max|out - ref| / max|ref|, both maxima over the whole tensor.

    The reference passes a case when err <= tol * scale; this returns the ratio so that
    ``max_rel_err(out, ref) <= tol`` decides exactly the same way:
      * a NaN anywhere in out (or ref) gives NaN, which fails every ``<=`` test;
      * an all-zero ref passes only an exactly-zero error (0 for err == 0, else inf);
      * out and ref must have one shape (no broadcasting of a transposed or flattened out);
      * an empty tensor has no error (0).
    """
    out = np.asarray(out, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    if out.shape != ref.shape:
        raise ValueError(f"max_rel_err: out {out.shape} and ref {ref.shape} differ in shape")
    if ref.size == 0:
        return 0.0
    err = float(np.max(np.abs(out - ref)))
    scale = float(np.max(np.abs(ref)))
    if np.isnan(err) or np.isnan(scale):
        return float("nan")
    if scale == 0.0:
        return 0.0 if err == 0.0 else float("inf")
    return err / scale


class Lcg:
    """csrc/micro/sanitize_gemm.cu:21-25: s = s * 1664525 + 1013904223 (mod 2^32)."""

    def __init__(self, seed: int):
        self.s = seed & 0xFFFFFFFF

    def next_block(self, count: int) -> np.ndarray:
        """The next `count` states, computed sequentially (uint32 arithmetic)."""
        out = np.empty(count, dtype=np.uint32)
        s = self.s
        for i in range(count):
            s = (s * 1664525 + 1013904223) & 0xFFFFFFFF
            out[i] = s
        self.s = s
        return out

    @staticmethod
    def to_uniform(states: np.ndarray) -> np.ndarray:
        """uniform() = ((s >> 8) / 2^24) * 2 - 1 in fp32."""
        return (((states >> np.uint32(8)).astype(np.float32) / np.float32(16777216.0)) * np.float32(2.0)
                - np.float32(1.0))


def lcg_workload(group_size: int, n: int = 128, k: int = 1024, ms=(1, 3, 8, 9, 16, 17, 33, 64, 65)):
    """csrc/micro/sanitize_gemm.cu:36-50: the reference's torch-free deterministic workload.

    Order of draws: q for all N*K (top 4 bits - 8), then scales fp16(0.01 + 0.02|u|),
    then for each M in turn x = fp16(u) [M, K].  Returns (q int8 [N, K],
    scales fp16 [N, K/G], packed int32 [N, K/8], {M: x fp16 [M, K]}).
    """
    rng = Lcg(group_size)
    q = ((rng.next_block(n * k) >> np.uint32(28)).astype(np.int32) - 8).astype(np.int8).reshape(n, k)
    u = Lcg.to_uniform(rng.next_block(n * (k // group_size)))
    scales = (np.float32(0.01) + np.float32(0.02) * np.abs(u)).astype(np.float16).reshape(n, k // group_size)
    packed = pack_int4(q)
    xs = {}
    for m in ms:
        xs[m] = Lcg.to_uniform(rng.next_block(m * k)).astype(np.float16).reshape(m, k)
    return q, scales, packed, xs


def seeded_case(m: int, n: int, k: int, group_size: int, seed: int):
    """Deterministic CPU inputs in the distribution of tests/test_gemm.py:27-33.

    W ~ 0.02 * N(0, 1) fp32 [N, K] quantized with quantize_weight; x ~ N(0, 1) fp16 [M, K].
    numpy's PCG64 replaces the reference's CUDA generator so any machine
    regenerates identical bytes.
    """
    rng = np.random.Generator(np.random.PCG64(seed))
    w = (rng.standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    x = rng.standard_normal((m, k), dtype=np.float32).astype(np.float16)
    packed, scales = quantize_weight(w, group_size)
    return w, x, packed, scales


def algorithmic_bytes(m: int, n: int, k: int, group_size: int) -> int:
    """bench/bench_gemm.py:80,98: packed + scales + x + y bytes."""
    return n * k // 2 + 2 * n * (k // group_size) + 2 * m * k + 2 * m * n


def gemm_flops(m: int, n: int, k: int) -> int:
    """kernelforge/bench_utils.py:209-210."""
    return 2 * m * n * k


def reorder_mfma16(packed: np.ndarray, scales: np.ndarray, group_size: int) -> tuple[np.ndarray, np.ndarray]:
    """Layout contract of kf_int4_reorder_mfma16 (include/kf_int4.h); no reference counterpart.

    packed int32 [N, K/8], scales fp16 [N, K/G] -> (packed_r int32 [ceil(N/16) * 16 * K/8],
    scales_r fp16 [ceil(N/16) * 16 * K/G]).  Pieces of 4 words in order (block b, super-step s,
    lane l): row min(16b + l%16, N-1), words 16s + 4(l/16) .. +3.  Scales in order (b, group j,
    column c): scales[min(16b + c, N-1), j].
    """
    n, kw = packed.shape
    k = kw * 8
    if k % 128 or group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError("reorder_mfma16 needs K % 128 == 0 and G in (64, 128)")
    nb, nss = -(-n // 16), k // 128
    rows = np.minimum(np.arange(nb * 16), n - 1)
    p = packed[rows].reshape(nb, 16, nss, 4, 4)           # [b, col, s, g, word]
    packed_r = np.ascontiguousarray(p.transpose(0, 2, 3, 1, 4)).reshape(-1)  # [b, s, g, col, word]
    sc = scales[rows].reshape(nb, 16, k // group_size)      # [b, col, j]
    scales_r = np.ascontiguousarray(sc.transpose(0, 2, 1)).reshape(-1)       # [b, j, col]
    return packed_r, scales_r
