"""group_sibling_linears_: which launches the sibling calls make (CPU; launches are stubbed).

The stubs record each launch and return tensors tagged with the weight and input they were
made from, so the tests check both the launch count and that every module still gets its own
output for its own input, whatever order or inputs the parent calls them with.
"""

from __future__ import annotations

import pytest
import torch
from torch import nn

from kernelforge import modules
from kernelforge import quantize as kq

K, G = 256, 128


def _lin(n: int, tag: int, bias: bool = False) -> modules.KFLinearInt4:
    qw = kq.quantize_weight(torch.full((n, K), 0.01 * tag), G)
    return modules.KFLinearInt4(qw, torch.full((n,), float(tag)) if bias else None)


class _Attn(nn.Module):
    def __init__(self):
        super().__init__()
        self.q_proj, self.k_proj, self.v_proj = _lin(64, 1), _lin(32, 2, bias=True), _lin(32, 3)
        self.o_proj = _lin(64, 4)


class _Mlp(nn.Module):
    def __init__(self):
        super().__init__()
        self.gate_proj, self.up_proj, self.down_proj = _lin(96, 5), _lin(96, 6), _lin(64, 7)


class _Block(nn.Module):
    def __init__(self):
        super().__init__()
        self.self_attn, self.mlp = _Attn(), _Mlp()


@pytest.fixture
def launches(monkeypatch):
    """Stubs for the two launch paths; each output is [*lead, N] filled with a tag of (weight, x)."""
    log = []

    def tag(x, packed):
        return float(packed.shape[0]) * 1000 + float(x.flatten()[0])

    def linear(x, packed, scales, group_size=128, bias=None):
        log.append(("single", packed.shape[0]))
        return torch.full((*x.shape[:-1], packed.shape[0]), tag(x, packed), dtype=torch.float32)

    def grouped(xs, packed, scales, group_size=128, biases=None):
        log.append(("grouped", tuple(p.shape[0] for p in packed)))
        assert biases is not None and len(biases) == len(xs)
        return [torch.full((*x.shape[:-1], p.shape[0]), tag(x, p), dtype=torch.float32) for x, p in zip(xs, packed)]

    monkeypatch.setattr(modules.ops, "int4_linear", linear)
    monkeypatch.setattr(modules.ops, "int4_linear_grouped", grouped)
    return log


def _x(v: float, m: int = 1):
    return torch.full((1, m, K), v, dtype=torch.float16)


def test_groups_found_and_state_dict_unchanged():
    blk = _Block()
    before = {k: v.clone() for k, v in blk.state_dict().items()}
    assert modules.group_sibling_linears_(blk) == 2
    a, m = blk.self_attn, blk.mlp
    assert a.q_proj._siblings is a.k_proj._siblings is a.v_proj._siblings is not None
    assert m.gate_proj._siblings is m.up_proj._siblings is not None
    assert a.o_proj._siblings is None and m.down_proj._siblings is None
    after = blk.state_dict()
    assert before.keys() == after.keys() and all(torch.equal(before[k], after[k]) for k in before)


def test_one_launch_per_sibling_round(launches):
    blk = _Block()
    modules.group_sibling_linears_(blk)
    a = blk.self_attn
    for step in range(3):
        x = _x(step + 1)
        q, k, v = a.q_proj(x), a.k_proj(x), a.v_proj(x)
        assert [t.shape[-1] for t in (q, k, v)] == [64, 32, 32]
        assert q[0, 0, 0] == 64 * 1000 + step + 1 and k[0, 0, 0] == 32 * 1000 + step + 1
    assert launches == [("grouped", (64, 32, 32))] * 3
    assert a.q_proj._siblings._x is None and a.q_proj._siblings._ys is None  # references dropped


def test_any_call_order_and_a_foreign_input(launches):
    blk = _Block()
    modules.group_sibling_linears_(blk)
    g, u = blk.mlp.gate_proj, blk.mlp.up_proj
    x1, x2 = _x(1.0), _x(2.0)
    assert u(x1)[0, 0, 0] == 96 * 1000 + 1   # up first: launches the group
    assert g(x1)[0, 0, 0] == 96 * 1000 + 1   # gate takes the waiting output
    assert launches == [("grouped", (96, 96))]
    g(x1)                                     # gate again on x1: nothing waits, new group
    assert launches[-1] == ("grouped", (96, 96))
    y = u(x2)                                 # up on another input while up's output waits
    assert y[0, 0, 0] == 96 * 1000 + 2 and launches[-1] == ("single", 96)
    assert g._siblings._pending == set()      # waiting output dropped
    same = torch.full((1, 1, K), 2.0, dtype=torch.float16)
    g(x2)
    assert u(same)[0, 0, 0] == 96 * 1000 + 2  # equal values, another object: runs on its own
    assert launches[-2:] == [("grouped", (96, 96)), ("single", 96)]


def test_ungrouped_and_wrong_dtype(launches):
    blk = _Block()
    assert blk.self_attn.q_proj(_x(1.0)).shape == (1, 1, 64) and launches == [("single", 64)]
    modules.group_sibling_linears_(blk)
    with pytest.raises(TypeError, match="fp16"):
        blk.self_attn.q_proj(torch.ones(1, 1, K))
    blk.self_attn.q_proj._siblings = None
    blk.self_attn.q_proj(_x(1.0))
    assert launches[-1] == ("single", 64)


def test_mismatched_siblings_are_not_grouped():
    blk = _Block()
    blk.self_attn.v_proj = modules.KFLinearInt4(kq.quantize_weight(torch.ones(32, 2 * K) * 0.01, G), None)
    blk.mlp.up_proj = modules.KFLinearInt4(kq.quantize_weight(torch.ones(96, K) * 0.01, 64), None)
    assert modules.group_sibling_linears_(blk) == 0


def test_input_updated_in_place_between_siblings_is_not_paired(launches):
    blk = _Block()
    modules.group_sibling_linears_(blk)
    g, u = blk.mlp.gate_proj, blk.mlp.up_proj
    x = _x(1.0)
    g(x)
    x.fill_(3.0)                          # same object, new contents: the waiting output is stale
    assert u(x)[0, 0, 0] == 96 * 1000 + 3
    assert launches == [("grouped", (96, 96)), ("single", 96)]
    with torch.inference_mode():          # no version counter: identity alone pairs the calls
        xi = _x(5.0)
        g(xi)
        assert u(xi)[0, 0, 0] == 96 * 1000 + 5
    assert launches[-1] == ("grouped", (96, 96))
