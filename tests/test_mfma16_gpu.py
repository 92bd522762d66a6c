"""MFMA-16 block copy of a weight (kf_int4_reorder_mfma16, kf_int4_gemm_mfma16) and the op-level
cache behind int4_gemm (needs a GPU).

The copy is a pure permutation, checked bit for bit against the oracle's statement of the layout
(oracle/int4_oracle.py:reorder_mfma16, itself pinned element by element in test_oracle.py).  The
GEMM reading it must equal the GEMM reading the public layout bit for bit: same dequantization,
same MFMA order, same fixed-order reduction.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kernelforge import _lib, ops
from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _weight(n: int, k: int, g: int, seed: int = 0):
    rng = np.random.default_rng(seed + n * 3 + k)
    packed, scales = o.quantize_weight((rng.standard_normal((n, k)) * 0.02).astype(np.float32), g)
    return packed, scales, torch.from_numpy(packed).to(DEV), torch.from_numpy(scales).to(DEV)


def _gemm_raw(x, dp, ds, g, copy=None):
    """kf_int4_gemm, or kf_int4_gemm_mfma16 with `copy`, straight through the C ABI."""
    lib = _lib.load()
    m, k = x.shape
    n = dp.shape[0]
    y = torch.empty(m, n, dtype=torch.float16, device=DEV)
    wsb = lib.kf_int4_gemm_workspace_bytes(m, n, k, g)
    ws = torch.empty(max(wsb, 16) // 4 + 1, dtype=torch.float32, device=DEV)
    stream = torch.cuda.current_stream().cuda_stream
    if copy is None:
        st = lib.kf_int4_gemm(x.data_ptr(), dp.data_ptr(), ds.data_ptr(), y.data_ptr(), ws.data_ptr(), wsb, m, n, k,
                              g, stream)
    else:
        st = lib.kf_int4_gemm_mfma16(x.data_ptr(), dp.data_ptr(), ds.data_ptr(), copy[0].data_ptr(),
                                     copy[1].data_ptr(), y.data_ptr(), ws.data_ptr(), wsb, m, n, k, g, stream)
    _lib.check(st, "gemm")
    return y


@pytest.mark.parametrize("n,k,g", [(1, 128, 128), (17, 256, 64), (100, 2048, 128), (5632, 2048, 128),
                                   (1536, 8960, 128), (2048, 5632, 64), (256, 1536, 64)])
def test_reorder_matches_oracle(n, k, g):
    packed, scales, dp, ds = _weight(n, k, g)
    pr, sr = ops.int4_reorder_mfma16(dp, ds, g)
    want_p, want_s = o.reorder_mfma16(packed, scales, g)
    assert np.array_equal(pr.cpu().numpy(), want_p)
    assert np.array_equal(sr.cpu().numpy().view(np.uint16), want_s.view(np.uint16))


# gate, wide_a and wide_b take two 16-column blocks per skinny workgroup on 256 CUs
# (SkinnyPlan::col_blocks; N is a multiple of 64 on the GEMM path, so those workgroups are whole).
LAYERS = {"qo": (2048, 2048), "kv": (256, 2048), "gate": (5632, 2048), "down": (2048, 5632),
          "qwen_down": (1536, 8960), "ragged": (320, 1152), "wide_a": (4160, 2048), "wide_b": (6016, 1024)}


@pytest.mark.parametrize("layer", list(LAYERS))
@pytest.mark.parametrize("g", [64, 128])
def test_gemm_with_copy_is_bit_identical(layer, g):
    """Every M of the skinny range (plus one tiled M, where the copy is not read)."""
    n, k = LAYERS[layer]
    packed, scales, dp, ds = _weight(n, k, g)
    copy = ops.int4_reorder_mfma16(dp, ds, g)
    skinny_seen = 0
    for m in (1, 2, 3, 5, 8, 9, 13, 16, 17, 24, 32, 64):
        x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half().to(DEV)
        ref = _gemm_raw(x, dp, ds, g)
        got = _gemm_raw(x, dp, ds, g, copy)
        assert torch.equal(got, ref), f"{layer} M={m}"
        skinny_seen += ops.gemm_plan(m, n, k, g)["kernel"] == "skinny"
    assert skinny_seen >= 5
    # and against the oracle at one M, so the check is not only self-consistency
    x = o.seeded_case(8, n, k, g, seed=3)[1]
    y = _gemm_raw(torch.from_numpy(x).to(DEV), dp, ds, g, copy).float().cpu().numpy()
    assert o.max_rel_err(y, o.linear_ref_fp32(x, packed, scales, g)) <= 2e-3


def test_op_cache_builds_reuses_and_invalidates():
    n, k, g = 2048, 2048, 128
    _, _, dp, ds = _weight(n, k, g)
    x = torch.randn(8, k, device=DEV).half()
    old = ops.MFMA16_CACHE
    try:
        ops.MFMA16_CACHE = False
        plain = ops.int4_gemm(x, dp, ds, g)
        assert getattr(dp, "_kf_mfma16", None) is None
        ops.MFMA16_CACHE = True
        y1 = ops.int4_gemm(x, dp, ds, g)
        first = getattr(dp, "_kf_mfma16")
        y2 = ops.int4_gemm(x, dp, ds, g)
        assert getattr(dp, "_kf_mfma16") is first  # reused
        assert torch.equal(y1, plain) and torch.equal(y2, plain)
        # an in-place update of the weight invalidates the copy
        packed2, scales2, dp2, ds2 = _weight(n, k, g, seed=9)
        dp.copy_(dp2)
        ds.copy_(ds2)
        y3 = ops.int4_gemm(x, dp, ds, g)
        assert getattr(dp, "_kf_mfma16") is not first
        assert torch.equal(y3, ops.int4_gemm(x, dp2, ds2, g))
        # a tiled-kernel M builds nothing
        _, _, dp3, ds3 = _weight(5632, 2048, g, seed=4)
        ops.int4_gemm(torch.randn(64, 2048, device=DEV).half(), dp3, ds3, g)
        assert getattr(dp3, "_kf_mfma16", None) is None
    finally:
        ops.MFMA16_CACHE = old


def test_default_builds_no_copy_but_uses_a_prepared_one():
    """The copy is opt-in: by default int4_gemm attaches nothing; a copy attached with
    prepare_mfma16 is read (same bits) and ignored once the weight is updated in place."""
    assert ops.MFMA16_CACHE is False
    n, k, g = 2048, 2048, 128
    _, _, dp, ds = _weight(n, k, g, seed=5)
    x = torch.randn(8, k, device=DEV).half()
    plain = ops.int4_gemm(x, dp, ds, g)
    assert getattr(dp, "_kf_mfma16", None) is None
    ops.prepare_mfma16(dp, ds, g)
    copy = getattr(dp, "_kf_mfma16")
    assert torch.equal(ops.int4_gemm(x, dp, ds, g), plain) and getattr(dp, "_kf_mfma16") is copy
    _, _, dp2, ds2 = _weight(n, k, g, seed=6)
    dp.copy_(dp2)
    ds.copy_(ds2)
    assert torch.equal(ops.int4_gemm(x, dp, ds, g), ops.int4_gemm(x, dp2, ds2, g))
    assert getattr(dp, "_kf_mfma16") is copy  # stale, not rebuilt without MFMA16_CACHE, not read


def test_graph_capture_uses_cached_copy(monkeypatch):
    monkeypatch.setattr(ops, "MFMA16_CACHE", True)
    n, k, g = 5632, 2048, 128
    _, _, dp, ds = _weight(n, k, g)
    static_x = torch.randn(4, k, device=DEV).half()
    eager = ops.int4_gemm(static_x, dp, ds, g)  # builds the copy outside capture
    assert getattr(dp, "_kf_mfma16", None) is not None
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        ops.int4_gemm(static_x, dp, ds, g)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        static_y = ops.int4_gemm(static_x, dp, ds, g)
    for i in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(static_y, eager), f"replay {i}"
        ops.int4_gemm(static_x, dp, ds, g)
        torch.cuda.synchronize()


def test_mfma16_rejections():
    lib = _lib.load()
    pb, sb = ctypes.c_size_t(), ctypes.c_size_t()
    assert lib.kf_int4_mfma16_sizes(100, 1152, 128, ctypes.byref(pb), ctypes.byref(sb)) == 0
    assert pb.value == 112 * 1152 // 2 and sb.value == 112 * 9 * 2
    assert lib.kf_int4_mfma16_sizes(100, 192, 64, None, None) != 0  # K % 128
    assert "multiple of 128" in _lib.last_error()
    _, _, dp, ds = _weight(64, 256, 128)
    stream = torch.cuda.current_stream().cuda_stream
    assert lib.kf_int4_reorder_mfma16(dp.data_ptr(), ds.data_ptr(), None, None, 64, 256, 128, stream) != 0
    with pytest.raises(TypeError):
        ops.int4_reorder_mfma16(dp.float(), ds, 128)


def test_inference_mode_weights_use_only_a_prepared_copy():
    """Inference tensors carry no version counter: no implicit copy; prepare_mfma16 opts in."""
    n, k, g = 2048, 2048, 128
    packed, scales, _, _ = _weight(n, k, g)
    with torch.inference_mode():
        dp = torch.from_numpy(packed).to(DEV)
        ds = torch.from_numpy(scales).to(DEV)
        x = torch.randn(8, k, device=DEV).half()
        plain = ops.int4_gemm(x, dp, ds, g)
        assert getattr(dp, "_kf_mfma16", None) is None
        ops.prepare_mfma16(dp, ds, g)
        assert getattr(dp, "_kf_mfma16", None) is not None
        assert torch.equal(ops.int4_gemm(x, dp, ds, g), plain)
