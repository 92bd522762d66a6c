"""The op boundary under tracers, on the CPU (no GPU, no kernel launch).

The reference's int4_linear always calls the registered op kernelforge::int4_matmul
(kernelforge/ops.py:277-302), so FakeTensorMode, make_fx and other dispatch-mode tooling see
the op and its fake impl.  The package's int4_linear skips the dispatcher for eager calls on
plain tensors only; these tests check that every tracer still gets the op: the fake impl's
shapes come back, make_fx records the op, and no device pointer of a fake tensor is read
(UserWarnings, which torch raises for data_ptr() on a FakeTensor, are errors here).
"""

from __future__ import annotations

import warnings

import pytest
import torch
from torch._subclasses.fake_tensor import FakeTensor, FakeTensorMode
from torch.fx.experimental.proxy_tensor import make_fx

from kernelforge import modules, ops
from kernelforge import quantize as kq

N, K, G = 5632, 2048, 128


@pytest.fixture(autouse=True)
def _warnings_are_errors():
    with warnings.catch_warnings():
        warnings.simplefilter("error", UserWarning)
        yield


def _fake(mode: FakeTensorMode, *shape, dtype=torch.float16):
    with mode:
        return torch.empty(*shape, dtype=dtype, device="cuda")


def _weight(mode, n=N, k=K, g=G):
    return _fake(mode, n, k // 8, dtype=torch.int32), _fake(mode, n, k // g)


def _ops_in(gm: torch.fx.GraphModule) -> list[str]:
    return [str(node.target) for node in gm.graph.nodes if node.op == "call_function"]


def test_int4_linear_under_fake_tensor_mode():
    mode = FakeTensorMode()
    p, s = _weight(mode)
    with mode:
        for lead in [(1,), (3,), (2, 3)]:
            x = torch.empty(*lead, K, dtype=torch.float16, device="cuda")
            y = ops.int4_linear(x, p, s, G)
            assert isinstance(y, FakeTensor) and y.shape == (*lead, N) and y.dtype == torch.float16
            assert y.device.type == "cuda"
        bias = torch.empty(N, dtype=torch.float16, device="cuda")
        assert ops.int4_linear(torch.empty(4, K, dtype=torch.float16, device="cuda"), p, s, G, bias).shape == (4, N)


def test_fake_inputs_outside_their_mode_take_the_op():
    """FakeTensors used with no mode on the stack are tensor subclasses: the op (and its fake impl
    under the tensors' own mode) runs, not a launch."""
    mode = FakeTensorMode()
    p, s = _weight(mode)
    x = _fake(mode, 2, K)
    assert ops._traced((x, p, s)) and torch._C._len_torch_dispatch_stack() == 0
    y = ops.int4_linear(x, p, s, G)
    assert isinstance(y, FakeTensor) and y.shape == (2, N)


def test_eager_plain_tensors_skip_the_dispatcher():
    plain = torch.zeros(2, 2)
    param = torch.nn.Parameter(torch.zeros(2, 2), requires_grad=False)
    assert not ops._traced((plain, param, None))
    with FakeTensorMode():
        assert ops._traced((plain,))


def test_grouped_and_module_under_fake_tensor_mode():
    mode = FakeTensorMode()
    p, s = _weight(mode)
    pk, sk = _weight(mode, 256, K)
    with mode:
        x = torch.empty(1, K, dtype=torch.float16, device="cuda")
        ys = ops.int4_linear_grouped([x, x, x], [p, pk, pk], [s, sk, sk], G)
        assert [tuple(y.shape) for y in ys] == [(1, N), (1, 256), (1, 256)]
        lin = modules.KFLinearInt4(kq.QuantizedWeight(p, s, G, (N, K)),
                                   torch.empty(N, dtype=torch.float16, device="cuda"))
        y = lin(torch.empty(2, 5, K, dtype=torch.float16, device="cuda"))
        assert isinstance(y, FakeTensor) and y.shape == (2, 5, N)
        with pytest.raises(TypeError, match="fp16"):
            lin(torch.empty(1, K, dtype=torch.float32, device="cuda"))


def test_validation_still_runs_first_under_tracing():
    """The reference's checks (same order, types, messages) run before the op in every mode."""
    mode = FakeTensorMode()
    p, s = _weight(mode)
    with mode:
        with pytest.raises(ValueError, match="K/8"):
            ops.int4_linear(torch.empty(1, K // 2, dtype=torch.float16, device="cuda"), p, s, G)
        with pytest.raises(TypeError, match="fp16 CUDA"):
            ops.int4_linear(torch.empty(1, K, dtype=torch.float16), p, s, G)
        with pytest.raises(ValueError, match="not a multiple of group_size"):
            ops.int4_linear(torch.empty(1, 200, dtype=torch.float16, device="cuda"),
                            torch.empty(N, 25, dtype=torch.int32, device="cuda"), s, G)


def test_make_fx_records_the_registered_op():
    mode = FakeTensorMode()
    p, s = _weight(mode)
    x = _fake(mode, 2, 3, K)
    b = _fake(mode, N)
    with mode:
        gm = make_fx(lambda a, pp, ss, bb: ops.int4_linear(a, pp, ss, G, bb))(x, p, s, b)
    assert "kernelforge.int4_matmul.default" in _ops_in(gm)
    out = [n for n in gm.graph.nodes if n.op == "output"][0].args[0]
    assert tuple(out.meta["val"].shape) == (2, 3, N)
    with mode:
        lin = modules.KFLinearInt4(kq.QuantizedWeight(p, s, G, (N, K)), None)
        gm = make_fx(lambda a: lin(a))(_fake(mode, 4, K))
    assert _ops_in(gm).count("kernelforge.int4_matmul.default") == 1
    with mode:
        gm = make_fx(lambda a, c: ops.int4_linear_grouped([a, c], [p, p], [s, s], G))(_fake(mode, 1, K),
                                                                                     _fake(mode, 1, K))
    assert "kernelforge.int4_matmul_grouped.default" in _ops_in(gm)


def test_fused_decode_ops_under_fake_tensor_mode():
    mode = FakeTensorMode()
    p, s = _weight(mode)
    with mode:
        x = torch.empty(1, 1, K, dtype=torch.float16, device="cuda")
        w = torch.empty(K, dtype=torch.float16, device="cuda")
        r = torch.empty(1, 1, N, dtype=torch.float16, device="cuda")
        assert ops.int4_linear_fused(x, p, s, G, norm_weight=w, residual=r).shape == (1, 1, N)
        assert ops.int4_linear_fused(x, p, s, G, up=x).shape == (1, 1, N)
        heads, kv_heads, d, seq = 32, 4, 64, 64
        n_qkv = (heads + 2 * kv_heads) * d
        pq, sq = torch.empty(n_qkv, K // 8, dtype=torch.int32, device="cuda"), \
            torch.empty(n_qkv, K // G, dtype=torch.float16, device="cuda")
        tab = torch.empty(seq, d, dtype=torch.float16, device="cuda")
        pos = torch.zeros(1, dtype=torch.int64, device="cuda")
        ck = torch.empty(kv_heads, d, seq, dtype=torch.float16, device="cuda")
        cv = torch.empty(kv_heads, seq, d, dtype=torch.float16, device="cuda")
        y = ops.int4_qkv_rope_cache(x, pq, sq, G, cos=tab, sin=tab, pos=pos, cache_k=ck, cache_v=cv, heads=heads,
                                    kv_heads=kv_heads, head_dim=d, norm_weight=w)
        assert y.shape == (1, 1, n_qkv)
        gm = make_fx(lambda a: ops.int4_linear_fused(a, p, s, G, norm_weight=w, residual=r))(x)
    assert "kernelforge.int4_linear_fused.default" in _ops_in(gm)


def test_launch_helpers_refuse_fake_tensors():
    """A direct call of the launch-level entry points with fake tensors raises before any pointer
    is read, instead of launching on a fake address."""
    mode = FakeTensorMode()
    p, s = _weight(mode)
    x = _fake(mode, 1, K)
    for fn in (ops._check_native, ops._check_native_each):
        with pytest.raises(RuntimeError, match="no device memory"):
            fn(x, p, s, G)
