"""On-device quantize + pack (kf_int4_quantize) against the oracle, bit for bit (needs a GPU).

The oracle restates the reference's CPU quantizer (kernelforge/quantize.py:61-105) and is pinned
by tests/test_oracle.py (KATs, exact-rational brute force on gaussian / tie / tiny / mixed
groups).  Here the GPU kernel must reproduce it exactly on: every layer shape of the benchmark,
fp32 / fp16 / bf16 inputs (converted exactly to fp32), both group sizes, ragged N, exact .5 ties,
the +-7 ends, tiny and all-zero groups, wide dynamic ranges, and the peaks for which
fl32(peak / 7) and fl32(peak * fl32(1/7)) round to different fp16 scales (the kernel must divide,
as the CPU does).
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from kernelforge import ops
from kernelforge import quantize as kq
from kernelforge.modules import KFLinearInt4, quantize_linears_
from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _assert_matches_oracle(w: torch.Tensor, group: int) -> None:
    """w on the CPU in its dtype; the oracle quantizes its exact fp32 value."""
    ref_packed, ref_scales = o.quantize_weight(w.float().numpy(), group)
    packed, scales = ops.int4_quantize(w.to(DEV), group)
    got_p, got_s = packed.cpu().numpy(), scales.cpu().numpy()
    bad = np.nonzero((got_p != ref_packed).any(axis=1) | (got_s.view(np.uint16) != ref_scales.view(np.uint16)).any(axis=1))[0]
    assert bad.size == 0, f"{bad.size} rows differ, first {bad[:5].tolist()}"


SHAPES = [(2048, 2048), (256, 2048), (5632, 2048), (2048, 5632), (1536, 8960), (8960, 1536), (1, 128), (3, 256),
          (9, 192), (129, 4160)]


# Every (shape, group) whose K the group divides (quantize_weight rejects the others; that
# rejection is tested on the CPU).
SHAPE_GROUPS = [(shape, group) for shape in SHAPES for group in (64, 128) if shape[1] % group == 0]


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("shape,group", SHAPE_GROUPS)
def test_quantize_matches_oracle(shape, group, dtype):
    n, k = shape
    g = torch.Generator().manual_seed(n * 131 + k + group)
    w = (torch.randn(n, k, generator=g) * 0.02).to(dtype)
    _assert_matches_oracle(w, group)


def test_quantize_crafted_groups():
    """Exact ties, the +-7 ends, tiny / zero / negative-zero groups, mixed ranges (G = 64)."""
    rows = []
    s = np.float32(0.5)  # absmax 3.5 gives the scale fp16(3.5 / 7) = 0.5 exactly
    ties = np.zeros(64, np.float32)
    ties[0] = 3.5
    ties[1:15] = (np.arange(-7, 7, dtype=np.float32) + np.float32(0.5)) * s  # w / s = j + .5: ties to even
    rows.append(ties)
    ends = np.zeros(64, np.float32)
    ends[:3] = [-3.5, 3.5, -3.25]  # w / s = -7, 7, -6.5
    rows.append(ends)
    tiny = np.full(64, 1e-6, np.float32)
    tiny[3] = -3e-6  # absmax / 7 < 2^-14: the scale clamps before the fp16 cast
    rows.append(tiny)
    rows.append(np.zeros(64, np.float32))                      # all-zero group: scale 1
    rows.append(np.full(64, -0.0, np.float32))                 # negative zeros
    rng = np.random.default_rng(11)
    for scale in (1e-4, 1.0, 30.0, 3000.0):
        rows.append((rng.standard_normal(64) * scale).astype(np.float32))
    w = torch.from_numpy(np.stack(rows))
    _assert_matches_oracle(w, 64)


def test_quantize_divides_like_the_cpu():
    """Peaks where fl32(p / 7) and fl32(p * fl32(1/7)) give different fp16 scales: the kernel
    must follow the CPU's true division (and so equal quantize_weight on the CPU)."""
    rng = np.random.default_rng(0)
    x = (rng.random(4_000_000, dtype=np.float32) * np.float32(0.2)).astype(np.float32)
    by_div = np.maximum(x / np.float32(7.0), np.float32(2**-14)).astype(np.float16)
    by_mul = np.maximum(x * np.float32(1.0 / 7.0), np.float32(2**-14)).astype(np.float16)
    peaks = x[by_div.view(np.uint16) != by_mul.view(np.uint16)][:256]
    assert peaks.size >= 64
    w = (rng.standard_normal((peaks.size, 128)) * 1e-4).astype(np.float32)
    w[:, 17] = peaks  # the group's absmax
    w = torch.from_numpy(w)
    _assert_matches_oracle(w, 128)
    cpu = kq.quantize_weight(w, 128)
    gpu = kq.quantize_weight(w.to(DEV), 128)  # routed to the kernel
    assert torch.equal(gpu.packed.cpu(), cpu.packed) and torch.equal(gpu.scales.cpu(), cpu.scales)


@pytest.mark.parametrize("group", [64, 128])
def test_quantize_near_half_integers(group):
    """Values within a few ulps of (j + 1/2) * s, for 300 scales s: the kernel's reciprocal
    product must fall back to the division wherever the two could round apart, including the
    values for which fl32(v / s) is exactly j + 1/2 although v / s is not (ties by double
    rounding, resolved to even)."""
    rng = np.random.default_rng(5)
    scales = np.unique(np.concatenate([
        (2.0 ** rng.uniform(-13, 9, 280)).astype(np.float16),  # normal fp16 scales
        np.float16([2**-14, 1.0, 0.5, 0.75, 1.5, 3.0, 65504 / 7 / 2]),
    ]).astype(np.float32))
    combos = [(j, n) for j in range(-7, 7) for n in range(-3, 4)]
    rows = []
    for s in scales:
        row = np.empty(256, np.float32)
        for g0 in range(0, 256, group):
            row[g0] = np.float32(7.0) * s  # absmax 7 s: the group's scale is s exactly
            for slot in range(1, group):
                j, n = combos[(g0 + slot) % len(combos)]
                v = np.float32((j + 0.5) * s)  # exact: 4 + 11 significant bits
                for _ in range(abs(n)):
                    v = np.nextafter(v, np.float32(np.inf) if n > 0 else np.float32(-np.inf), dtype=np.float32)
                row[g0 + slot] = v
        rows.append(row)
    w = np.stack(rows)
    # The crafted set holds double-rounding ties: v != (j + 1/2) s, yet fl32(v / s) = j + 1/2.
    q = w / np.repeat(scales[:, None], 256, axis=1)
    half = np.abs(q - np.floor(q)) == np.float32(0.5)
    exact_half = np.zeros_like(half)
    for i, s in enumerate(scales):
        exact_half[i] = (np.floor(q[i]) + 0.5).astype(np.float32) * s == w[i]
    assert (half & ~exact_half).sum() > 100, "no double-rounding ties in the crafted values"
    _assert_matches_oracle(torch.from_numpy(w), group)


def test_quantize_noncontiguous_and_offset_inputs():
    base = torch.randn(64, 520, device=DEV) * 0.02
    view = base[:, 4:516]  # non-contiguous, storage offset of 16 bytes
    packed, scales = ops.int4_quantize(view, 128)
    ref_p, ref_s = o.quantize_weight(view.cpu().numpy().astype(np.float32), 128)
    assert np.array_equal(packed.cpu().numpy(), ref_p)
    assert np.array_equal(scales.cpu().numpy().view(np.uint16), ref_s.view(np.uint16))


def test_quantize_rejections():
    with pytest.raises(ValueError, match="not a multiple of group_size"):
        ops.int4_quantize(torch.zeros(16, 200, device=DEV), 128)
    with pytest.raises(ValueError, match="group_size"):
        ops.int4_quantize(torch.zeros(16, 256, device=DEV), 32)
    with pytest.raises(ValueError, match="2-D"):
        ops.int4_quantize(torch.zeros(4, 16, 256, device=DEV), 128)
    with pytest.raises(TypeError, match="CUDA"):
        ops.int4_quantize(torch.zeros(16, 256), 128)
    with pytest.raises(TypeError, match="float32, float16 and bfloat16"):
        ops.int4_quantize(torch.zeros(16, 256, device=DEV, dtype=torch.float64), 128)


def test_quantize_linears_on_gpu_equals_cpu():
    """quantize_linears_ on a model that lives on the GPU produces the CPU's buffers."""
    torch.manual_seed(5)

    class Block(nn.Module):
        def __init__(self):
            super().__init__()
            self.q_proj = nn.Linear(256, 256, bias=False)
            self.gate_proj = nn.Linear(256, 512, bias=True)

    cpu_model, gpu_model = Block(), Block()
    gpu_model.load_state_dict(cpu_model.state_dict())
    gpu_model = gpu_model.to(DEV)
    assert quantize_linears_(cpu_model, 128, ("q_proj", "gate_proj")) == 2
    assert quantize_linears_(gpu_model, 128, ("q_proj", "gate_proj")) == 2
    for name in ("q_proj", "gate_proj"):
        a, b = getattr(cpu_model, name), getattr(gpu_model, name)
        assert isinstance(b, KFLinearInt4)
        assert torch.equal(a.packed, b.packed.cpu()) and torch.equal(a.scales, b.scales.cpu())
