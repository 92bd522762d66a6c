"""The fused decode GEMV (kf_int4_gemv_fused / ops.int4_linear_fused) on the GPU.

* residual epilogue: bit-identical to ``residual + int4_linear(x)`` (also in place, y == residual);
* RMSNorm and SwiGLU prologues: against the FP32 oracle fed the prologue restated in float64 on
  the CPU (RMSNorm: x * (mean(x^2) + eps)^-1/2 * w rounded to fp16; SwiGLU: fp16(fp16(silu(g)) * u)),
  at the suite's rule max|out - ref| <= 2e-3 * max|ref|, and against the torch ops they replace;
* shapes the fused launch does not take (M > 1, K > 10240) run the torch composition;
* HIP-graph replays equal eager calls.
"""

from __future__ import annotations

import ctypes

import numpy as np
import pytest
import torch

from kernelforge import _lib, ops
from oracle import int4_oracle as o

pytestmark = pytest.mark.gpu

REL_TOL = 2e-3
DEV = "cuda"
G = 128
# (N, K): TinyLlama q|k|v, o, gate|up, down; Qwen2.5 q, down; a ragged N; K at the fused limit.
SHAPES = [(2560, 2048), (2048, 2048), (11264, 2048), (2048, 5632), (1536, 1536), (1536, 8960), (1000, 2048),
          (256, 10240)]


def _rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def _weight(n: int, k: int, g: int = G):
    w = (_rng(n * 131 + k).standard_normal((n, k), dtype=np.float32) * np.float32(0.02)).astype(np.float32)
    packed, scales = o.quantize_weight(w, g)
    return packed, scales, torch.from_numpy(packed).to(DEV), torch.from_numpy(scales).to(DEV)


def _h(a: np.ndarray) -> torch.Tensor:
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float16)).to(DEV)


def _rmsnorm_ref16(x16: np.ndarray, w16: np.ndarray, eps: float) -> np.ndarray:
    x = x16.astype(np.float64)
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return (x * r * w16.astype(np.float64)).astype(np.float16)


def _swiglu_ref16(g16: np.ndarray, u16: np.ndarray) -> np.ndarray:
    g = g16.astype(np.float64)
    s16 = (g / (1.0 + np.exp(-g))).astype(np.float16)
    return (s16.astype(np.float64) * u16.astype(np.float64)).astype(np.float16)


def _assert_close(out: torch.Tensor, ref: np.ndarray, what: str) -> None:
    err = o.max_rel_err(out.float().cpu().numpy(), ref)
    assert err <= REL_TOL, f"{what}: max rel err {err:.3e} > {REL_TOL}"


@pytest.mark.parametrize("n,k", SHAPES)
def test_residual_epilogue_bit_identical(n, k):
    _, _, dp, ds = _weight(n, k)
    x = _h(_rng(n + k).standard_normal((1, k)))
    r = _h(_rng(n + k + 1).standard_normal((1, n)) * 4)
    got = ops.int4_linear_fused(x, dp, ds, G, residual=r)
    want = r + ops.int4_linear(x, dp, ds, G)
    assert torch.equal(got, want)
    # the same call through the C ABI with y == residual (in place)
    y = r.clone()
    lib = _lib.load()
    st = lib.kf_int4_gemv_fused(x.data_ptr(), dp.data_ptr(), ds.data_ptr(), y.data_ptr(), 1, n, k, G,
                                _lib.KF_PROLOGUE_NONE, None, ctypes.c_float(0.0), y.data_ptr(),
                                torch.cuda.current_stream().cuda_stream)
    _lib.check(st, "int4_gemv_fused")
    assert torch.equal(y, want)
    # no prologue, no residual: exactly int4_linear
    assert torch.equal(ops.int4_linear_fused(x, dp, ds, G), ops.int4_linear(x, dp, ds, G))


@pytest.mark.parametrize("n,k", SHAPES)
def test_rmsnorm_prologue(n, k):
    packed, scales, dp, ds = _weight(n, k)
    x16 = (_rng(n + 2 * k).standard_normal((1, k)) * 3).astype(np.float16)
    w16 = (_rng(k + 5).uniform(0.5, 1.5, k)).astype(np.float16)
    eps = 1e-5
    got = ops.int4_linear_fused(_h(x16), dp, ds, G, norm_weight=_h(w16), eps=eps)
    _assert_close(got, o.linear_ref_fp32(_rmsnorm_ref16(x16, w16, eps), packed, scales, G), "rmsnorm vs oracle")
    xn = torch.nn.functional.rms_norm(_h(x16), (k,), _h(w16), eps)
    _assert_close(got, ops.int4_linear(xn, dp, ds, G).float().cpu().numpy(), "rmsnorm vs torch")


@pytest.mark.parametrize("n,k", SHAPES)
def test_swiglu_prologue(n, k):
    packed, scales, dp, ds = _weight(n, k)
    g16 = (_rng(3 * n + k).standard_normal((1, k)) * 2).astype(np.float16)
    u16 = _rng(5 * n + k).standard_normal((1, k)).astype(np.float16)
    got = ops.int4_linear_fused(_h(g16), dp, ds, G, up=_h(u16))
    _assert_close(got, o.linear_ref_fp32(_swiglu_ref16(g16, u16), packed, scales, G), "swiglu vs oracle")
    xt = torch.nn.functional.silu(_h(g16)) * _h(u16)
    want = ops.int4_linear(xt, dp, ds, G)
    _assert_close(got, want.float().cpu().numpy(), "swiglu vs torch")


def test_prologue_plus_residual():
    n, k = 2048, 5632
    packed, scales, dp, ds = _weight(n, k)
    g16 = (_rng(11).standard_normal((1, k)) * 2).astype(np.float16)
    u16 = _rng(12).standard_normal((1, k)).astype(np.float16)
    r = _h(_rng(13).standard_normal((1, n)))
    got = ops.int4_linear_fused(_h(g16), dp, ds, G, up=_h(u16), residual=r)
    assert torch.equal(got, r + ops.int4_linear_fused(_h(g16), dp, ds, G, up=_h(u16)))
    n, k = 11264, 2048
    _, _, dp, ds = _weight(n, k)
    x, w, r = _h(_rng(14).standard_normal((1, k))), _h(_rng(15).uniform(0.5, 1.5, k)), _h(_rng(16).standard_normal((1, n)))
    got = ops.int4_linear_fused(x, dp, ds, G, norm_weight=w, residual=r)
    assert torch.equal(got, r + ops.int4_linear_fused(x, dp, ds, G, norm_weight=w))


def test_group_size_64_and_leading_dims():
    n, k = 2048, 2048
    packed, scales, dp, ds = _weight(n, k, 64)
    x16 = _rng(21).standard_normal((1, 1, k)).astype(np.float16)
    w16 = _rng(22).uniform(0.5, 1.5, k).astype(np.float16)
    got = ops.int4_linear_fused(_h(x16), dp, ds, 64, norm_weight=_h(w16))
    assert got.shape == (1, 1, n)
    _assert_close(got.view(1, n), o.linear_ref_fp32(_rmsnorm_ref16(x16.reshape(1, k), w16, 1e-5), packed, scales, 64),
                  "G=64")


@pytest.mark.parametrize("m,k", [(2, 2048), (5, 2048), (1, 12288)])
def test_other_sizes_run_the_torch_composition(m, k):
    n = 512
    _, _, dp, ds = _weight(n, k)
    x, w = _h(_rng(31).standard_normal((m, k))), _h(_rng(32).uniform(0.5, 1.5, k))
    u, r = _h(_rng(33).standard_normal((m, k))), _h(_rng(34).standard_normal((m, n)))
    got = ops.int4_linear_fused(x, dp, ds, G, norm_weight=w, residual=r)
    assert torch.equal(got, r + ops.int4_linear(torch.nn.functional.rms_norm(x, (k,), w, 1e-5), dp, ds, G))
    got = ops.int4_linear_fused(x, dp, ds, G, up=u)
    assert torch.equal(got, ops.int4_linear(torch.nn.functional.silu(x) * u, dp, ds, G))


def test_misaligned_operands_take_the_composition():
    """x or the SwiGLU up operand 2 bytes off a 16-byte boundary (one-row views into a larger
    buffer): the launch's LDS copies cannot take them, so the result is the torch composition's."""
    n, k = 2048, 2048
    _, _, dp, ds = _weight(n, k)
    buf = _h(_rng(51).standard_normal((1, k + 8)))
    x = buf[:, 1:k + 1]
    assert x.is_contiguous() and x.data_ptr() % 16 == 2
    w = _h(_rng(52).uniform(0.5, 1.5, k))
    got = ops.int4_linear_fused(x, dp, ds, G, norm_weight=w)
    assert torch.equal(got, ops.int4_linear(torch.nn.functional.rms_norm(x, (k,), w, 1e-5), dp, ds, G))
    g = _h(_rng(53).standard_normal((1, k)))
    up = buf[:, 1:k + 1]
    r = _h(_rng(54).standard_normal((1, n)))
    got = ops.int4_linear_fused(g, dp, ds, G, up=up, residual=r)
    assert torch.equal(got, r + ops.int4_linear(torch.nn.functional.silu(g) * up, dp, ds, G))


def test_graph_replays_equal_eager():
    n, k = 2048, 5632
    _, _, dp, ds = _weight(n, k)
    g, u, r = (_h(_rng(41 + i).standard_normal(s)) for i, s in enumerate([(1, k), (1, k), (1, n)]))
    eager = ops.int4_linear_fused(g, dp, ds, G, up=u, residual=r)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        ops.int4_linear_fused(g, dp, ds, G, up=u, residual=r)
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = ops.int4_linear_fused(g, dp, ds, G, up=u, residual=r)
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager)
        assert torch.equal(ops.int4_linear_fused(g, dp, ds, G, up=u, residual=r), eager)


def test_argument_errors():
    _, _, dp, ds = _weight(2048, 2048)
    x = _h(_rng(51).standard_normal((1, 2048)))
    with pytest.raises(ValueError, match="not both"):
        ops.int4_linear_fused(x, dp, ds, G, norm_weight=x[0], up=x)
    with pytest.raises(ValueError, match="norm_weight must be"):
        ops.int4_linear_fused(x, dp, ds, G, norm_weight=x[0, :100])
    with pytest.raises(ValueError, match="residual must be"):
        ops.int4_linear_fused(x, dp, ds, G, residual=x.float())


def _rope_tables(s: int, d: int):
    inv = 1.0 / (10000.0 ** (torch.arange(0, d, 2, dtype=torch.float32) / d))
    f = torch.outer(torch.arange(s, dtype=torch.float32), inv)
    return torch.cat([f, f], -1).cos().half().to(DEV), torch.cat([-f.sin(), f.sin()], -1).half().to(DEV)


@pytest.mark.parametrize("heads,kv_heads,d,k,with_norm", [(32, 4, 64, 2048, True), (12, 2, 128, 1536, False),
                                                           (32, 4, 64, 2048, False)])
def test_qkv_rope_cache(heads, kv_heads, d, k, with_norm):
    """q|k|v GEMV with RoPE and the cache writes in its epilogue, against the unfused steps: the
    GEMV (bit-identical v), torch's x * cos + swap_halves(x) * sin on its fp16 output, index writes."""
    s_max = 48
    n = (heads + 2 * kv_heads) * d
    _, _, dp, ds = _weight(n, k)
    x = _h(_rng(61).standard_normal((1, 1, k)))
    w = _h(_rng(62).uniform(0.5, 1.5, k)) if with_norm else None
    cos, sin = _rope_tables(s_max, d)
    for p in (0, 17, s_max - 1):
        pos = torch.tensor([p], dtype=torch.int64, device=DEV)
        ck = _h(_rng(63 + p).standard_normal((kv_heads, d, s_max)))
        cv = _h(_rng(64 + p).standard_normal((kv_heads, s_max, d)))
        ck0, cv0 = ck.clone(), cv.clone()
        y = ops.int4_qkv_rope_cache(x, dp, ds, G, cos=cos, sin=sin, pos=pos, cache_k=ck, cache_v=cv, heads=heads,
                                    kv_heads=kv_heads, head_dim=d, norm_weight=w)
        base = ops.int4_linear_fused(x, dp, ds, G, norm_weight=w).view(n)
        nqk = (heads + kv_heads) * d
        assert torch.equal(y.view(n)[nqk:], base[nqk:])                       # v: the GEMV's bits
        qk = base[:nqk].view(heads + kv_heads, d)
        rot = torch.addcmul(qk * cos[p], torch.cat([qk[:, d // 2:], qk[:, :d // 2]], -1), sin[p])
        got = y.view(n)[:nqk].view(heads + kv_heads, d)
        # The epilogue rounds as torch's fp16 ops do: fp16(x * cos), then fp16(that + partner * sin)
        # with the fp16 x fp16 product exact in fp32, so it equals the restatement bit for bit.
        assert torch.equal(got, rot), (got.float() - rot.float()).abs().max().item()
        # caches: position p holds exactly what y holds, everything else is untouched
        kk = got[heads:]                                                       # [kv_heads, d]
        assert torch.equal(ck[:, :, p], kk)
        assert torch.equal(cv[:, p, :], y.view(n)[nqk:].view(kv_heads, d))
        ck[:, :, p] = ck0[:, :, p]
        cv[:, p, :] = cv0[:, p, :]
        assert torch.equal(ck, ck0) and torch.equal(cv, cv0)


def test_qkv_rope_position_outside_cache_writes_no_cache():
    heads, kv_heads, d, k, s_max = 8, 2, 64, 1024, 16
    n = (heads + 2 * kv_heads) * d
    _, _, dp, ds = _weight(n, k)
    x = _h(_rng(71).standard_normal((1, k)))
    cos, sin = _rope_tables(s_max, d)
    ck = _h(_rng(72).standard_normal((kv_heads, d, s_max)))
    cv = _h(_rng(73).standard_normal((kv_heads, s_max, d)))
    ck0, cv0 = ck.clone(), cv.clone()
    for p in (s_max, -1):
        pos = torch.tensor([p], dtype=torch.int64, device=DEV)
        y = ops.int4_qkv_rope_cache(x, dp, ds, G, cos=cos, sin=sin, pos=pos, cache_k=ck, cache_v=cv, heads=heads,
                                    kv_heads=kv_heads, head_dim=d)
        assert torch.isfinite(y.float()).all()
        assert torch.equal(ck, ck0) and torch.equal(cv, cv0)


def test_qkv_rope_graph_replays_equal_eager():
    heads, kv_heads, d, k, s_max = 32, 4, 64, 2048, 40
    n = (heads + 2 * kv_heads) * d
    _, _, dp, ds = _weight(n, k)
    x, w = _h(_rng(81).standard_normal((1, k))), _h(_rng(82).uniform(0.5, 1.5, k))
    cos, sin = _rope_tables(s_max, d)
    pos = torch.tensor([5], dtype=torch.int64, device=DEV)
    ck = torch.zeros(kv_heads, d, s_max, dtype=torch.float16, device=DEV)
    cv = torch.zeros(kv_heads, s_max, d, dtype=torch.float16, device=DEV)

    def call():
        return ops.int4_qkv_rope_cache(x, dp, ds, G, cos=cos, sin=sin, pos=pos, cache_k=ck, cache_v=cv, heads=heads,
                                       kv_heads=kv_heads, head_dim=d, norm_weight=w)

    eager = call()
    ck_e, cv_e = ck.clone(), cv.clone()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        call()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        out = call()
    for step in range(3):
        ck.zero_()
        cv.zero_()
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager) and torch.equal(ck, ck_e) and torch.equal(cv, cv_e), step
