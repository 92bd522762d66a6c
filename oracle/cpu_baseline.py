"""The reference's CPU FP32 dequant + matmul path, restated in torch.  TEST INFRASTRUCTURE ONLY.

Timed by bench.py's ``cpu_baseline`` leg (and checked against the numpy oracle in
tests/test_oracle.py); the product never imports it.  It follows the reference's own torch
code, which runs its elementwise ops and the matmul on all intra-op threads:

  * ``dequantize(qw, torch.float32)``: unpack the nibbles, ``q.float() * scales`` per group
    (kernelforge/quantize.py:88-97, 108-114);
  * ``x.float() @ W_hat.T`` (tests/test_gemm.py:32).

Two variants are timed: the whole path per call (unpack + dequant + matmul, what a CPU user of
the reference pays per call), and the matmul alone on a W_hat dequantized once.
"""

from __future__ import annotations

import torch

from oracle.int4_oracle import NIBBLE_K

# k offset j of a word sits at nibble position _POS_OF_K[j] (inverse of NIBBLE_K).
_POS_OF_K = [NIBBLE_K.index(j) for j in range(8)]


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """int32 [N, K/8] -> int8 [N, K] (kernelforge/quantize.py:88-97)."""
    n, kw = packed.shape
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    nib = (packed.unsqueeze(-1) >> shifts) & 0xF          # [N, K/8, 8] by nibble position
    return (nib[..., _POS_OF_K] - 8).to(torch.int8).reshape(n, kw * 8)


def dequantize_fp32(packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """W_hat = q * s in fp32 [N, K] (kernelforge/quantize.py:114; exact)."""
    q = unpack_int4(packed)
    n, k = q.shape
    return (q.view(n, k // group_size, group_size).float() * scales.float().unsqueeze(-1)).reshape(n, k)


def linear_fp32(x16: torch.Tensor, packed: torch.Tensor, scales: torch.Tensor, group_size: int) -> torch.Tensor:
    """y = x.float() @ dequantize(qw, float32).T, fp32 [M, N] (tests/test_gemm.py:32)."""
    return x16.float() @ dequantize_fp32(packed, scales, group_size).T


def matmul_only(x16: torch.Tensor, w_hat: torch.Tensor) -> torch.Tensor:
    """The matmul of linear_fp32 on a W_hat dequantized beforehand."""
    return x16.float() @ w_hat.T
