"""Group-wise symmetric INT4 weight format consumed by the MI355X int4_linear kernels.

Public API and format follow the reference module ``kernelforge/quantize.py``
(``QuantizedWeight`` :38-47, ``quantize_int4`` :61-71, ``pack_int4`` :74-85,
``unpack_int4`` :88-97, ``quantize_weight`` :100-105, ``dequantize`` :108-114,
``quantization_error`` :117-126), so ``quantize_linears_`` and any caller that
stores ``(packed, scales)`` keep working unchanged.

Format (nn.Linear convention, W is [N, K] and y = x @ W^T):

* ``scales`` fp16 [N, K/G]: per output row n and group g of G consecutive k,
  ``s = fp16(max(absmax/7, 2^-14))`` and ``s = 1`` for an all-zero group.
* ``q = clamp(rint(w / s), -8, 7)`` with w and s in fp32 and ties to even.
* ``packed`` int32 [N, K/8]: word j of row n stores ``u = q + 8`` for
  k = 8j .. 8j+7, nibble position p (bits 4p..4p+3) holding k offset
  ``(0, 2, 4, 6, 1, 3, 5, 7)[p]``.  Shifting the word right by 4i and masking
  with 0x000F000F therefore leaves the pair (k 2i, k 2i+1) in the two 16-bit
  halves, which is what the GPU unpack relies on.

This module is the format producer.  ``quantize_weight`` of a weight on a GPU
runs the gfx950 quantize + pack kernel (``kernelforge.ops.int4_quantize``),
bit-identical to the torch path below on the CPU; every other function runs
wherever its tensor lives, with torch elementwise ops.  The GEMV/GEMM kernels
never call this module.
"""

from __future__ import annotations

from dataclasses import dataclass

import torch

DEFAULT_GROUP_SIZE = 128
SUPPORTED_GROUP_SIZES = (64, 128)

# Nibble position p holds k offset NIBBLE_K[p] of an 8-weight word.
NIBBLE_K = (0, 2, 4, 6, 1, 3, 5, 7)
# Inverse map: k offset -> nibble position.
K_NIBBLE = tuple(NIBBLE_K.index(k) for k in range(8))

_FP16_TINY = float(torch.finfo(torch.float16).tiny)  # 2^-14, smallest normal fp16


@dataclass
class QuantizedWeight:
    """Packed INT4 weight: int32 nibbles [N, K/8] plus fp16 group scales [N, K/G]."""

    packed: torch.Tensor
    scales: torch.Tensor
    group_size: int
    shape: tuple[int, int]

    @property
    def nbytes(self) -> int:
        return 4 * self.packed.numel() + 2 * self.scales.numel()


def _validate(weight: torch.Tensor, group_size: int) -> tuple[int, int]:
    # Same checks and messages as kernelforge/quantize.py:50-58.
    if weight.dim() != 2:
        raise ValueError(f"weight must be 2-D [N, K], got shape {tuple(weight.shape)}")
    if group_size not in SUPPORTED_GROUP_SIZES:
        raise ValueError(f"group_size must be one of {SUPPORTED_GROUP_SIZES}, got {group_size}")
    rows, cols = weight.shape
    if cols % group_size:
        raise ValueError(f"K={cols} is not a multiple of group_size={group_size}. "
                         "Pad K or pick another group size.")
    return rows, cols


def quantize_int4(weight: torch.Tensor, group_size: int = DEFAULT_GROUP_SIZE) -> tuple[torch.Tensor, torch.Tensor]:
    """(q int8 [N, K] in [-8, 7], scales fp16 [N, K/G]); reference quantize.py:61-71."""
    rows, cols = _validate(weight, group_size)
    groups = weight.float().reshape(rows, cols // group_size, group_size)
    peak = groups.abs().amax(dim=2, keepdim=True)
    # The scale is rounded to fp16 first so q is computed against the exact
    # value the kernels multiply by.
    s16 = torch.clamp(peak / 7.0, min=_FP16_TINY).half()
    s = torch.where(peak == 0, torch.ones_like(peak), s16.float())
    q = (groups / s).round().clamp(-8, 7).to(torch.int8)
    return q.reshape(rows, cols), s.half().reshape(rows, cols // group_size)


def pack_int4(q: torch.Tensor) -> torch.Tensor:
    """int8 [N, K] in [-8, 7] -> int32 [N, K/8]; reference quantize.py:74-85."""
    if q.dim() != 2 or q.shape[1] % 8:
        raise ValueError(f"q must be [N, K] with K a multiple of 8, got {tuple(q.shape)}")
    if int(q.min()) < -8 or int(q.max()) > 7:
        raise ValueError("q values must lie in [-8, 7]")
    rows, cols = q.shape
    nib = (q.to(torch.int32) + 8).reshape(rows, cols // 8, 8)
    # Gather the k offsets into nibble order, then shift each into place.
    ordered = nib[..., list(NIBBLE_K)]
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=q.device)
    # Nibbles occupy disjoint bits, so the sum equals the bitwise OR.  Summing
    # in int64 avoids signed overflow when the top nibble is >= 8.
    word = (ordered.to(torch.int64) << shifts.to(torch.int64)).sum(dim=-1)
    word = torch.where(word >= 2**31, word - 2**32, word)
    return word.to(torch.int32)


def unpack_int4(packed: torch.Tensor) -> torch.Tensor:
    """Inverse of pack_int4: int32 [N, K/8] -> int8 [N, K]; reference quantize.py:88-97."""
    rows, words = packed.shape
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=packed.device)
    nib = (packed.unsqueeze(-1) >> shifts) & 0xF  # [rows, words, nibble position]
    q = nib[..., list(K_NIBBLE)].to(torch.int8) - 8
    return q.reshape(rows, words * 8)


_KERNEL_DTYPES = (torch.float32, torch.float16, torch.bfloat16)


def quantize_weight(weight: torch.Tensor, group_size: int = DEFAULT_GROUP_SIZE) -> QuantizedWeight:
    """Quantize and pack an nn.Linear weight [N, K]; reference quantize.py:100-105.

    A weight on a GPU in fp32 / fp16 / bf16 goes through the quantize kernel, which
    divides exactly as the CPU does (torch's GPU division by the scalar 7 would multiply
    by a rounded 1/7), so the result is the same bit for bit wherever the weight lives.
    """
    rows, cols = _validate(weight, group_size)
    if weight.is_cuda and weight.dtype in _KERNEL_DTYPES:
        from kernelforge import ops  # deferred: ops loads the HIP library

        packed, scales = ops.int4_quantize(weight, group_size)
        return QuantizedWeight(packed=packed, scales=scales, group_size=group_size, shape=(rows, cols))
    q, scales = quantize_int4(weight, group_size)
    return QuantizedWeight(packed=pack_int4(q).contiguous(), scales=scales.contiguous(),
                           group_size=group_size, shape=(rows, cols))


def dequantize(qw: QuantizedWeight, dtype: torch.dtype = torch.float16) -> torch.Tensor:
    """W_hat [N, K] = q * s; reference quantize.py:108-114.

    fp16 gives fp16(q * s) with one round-to-nearest-even (the product of a
    4-bit integer and an fp16 scale is exact before that rounding); fp32 gives
    the exact product.
    """
    rows, cols = qw.shape
    q = unpack_int4(qw.packed).reshape(rows, cols // qw.group_size, qw.group_size)
    if dtype == torch.float16:
        return (q.half() * qw.scales.unsqueeze(-1)).reshape(rows, cols)
    return (q.float() * qw.scales.float().unsqueeze(-1)).reshape(rows, cols).to(dtype)


def quantization_error(weight: torch.Tensor, qw: QuantizedWeight) -> dict:
    """Error of the INT4 approximation; reference quantize.py:117-126."""
    w = weight.float()
    err = dequantize(qw, torch.float32) - w
    return {
        "max_abs_err": err.abs().max().item(),
        "rmse": err.square().mean().sqrt().item(),
        "rel_fro_err": (err.norm() / w.norm().clamp_min(1e-30)).item(),
        "bits_per_weight": 8.0 * qw.nbytes / w.numel(),
    }
