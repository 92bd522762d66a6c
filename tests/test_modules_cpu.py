"""KFLinearInt4 / quantize_linears_ on the CPU (no launch): the module contract a checkpoint and a
model swap depend on (reference kernelforge/modules.py:19-65).

quantize_linears_ swaps exactly the decoder linears by attribute name and leaves lm_head alone;
each KFLinearInt4 keeps ``packed`` int32 [N, K/8], ``scales`` fp16 [N, K/G] and ``bias`` fp16 [N]
(no bias entry for a linear without one) as its state, with the oracle's packed bytes; a state
dict round-trips into a module built from another weight; activations other than fp16 are
refused before any kernel is reached.
"""

from __future__ import annotations

import numpy as np
import pytest
import torch
from torch import nn

from kernelforge.modules import DECODER_LINEARS, KFLinearInt4, quantize_linears_
from oracle import int4_oracle as o


class _Block(nn.Module):
    def __init__(self, hidden: int, inter: int, bias: bool):
        super().__init__()
        for name in ("q_proj", "k_proj", "v_proj", "o_proj"):
            setattr(self, name, nn.Linear(hidden, hidden, bias=bias))
        self.gate_proj = nn.Linear(hidden, inter, bias=False)
        self.up_proj = nn.Linear(hidden, inter, bias=False)
        self.down_proj = nn.Linear(inter, hidden, bias=bias)
        self.lm_head = nn.Linear(hidden, 64, bias=False)


@pytest.mark.parametrize("bias", [False, True])
@pytest.mark.parametrize("group", [64, 128])
def test_swap_buffers_and_packed_bytes(bias, group):
    torch.manual_seed(3)
    blk = _Block(256, 384, bias)
    weights = {n: getattr(blk, n).weight.detach().clone() for n in DECODER_LINEARS}
    biases = {n: getattr(blk, n).bias for n in DECODER_LINEARS}
    assert quantize_linears_(blk, group) == 7
    assert isinstance(blk.lm_head, nn.Linear) and not isinstance(blk.lm_head, KFLinearInt4)
    for name in DECODER_LINEARS:
        lin = getattr(blk, name)
        assert isinstance(lin, KFLinearInt4)
        n, k = weights[name].shape
        assert (lin.out_features, lin.in_features, lin.group_size) == (n, k, group)
        assert lin.extra_repr() == f"in_features={k}, out_features={n}, group_size={group}, int4"
        sd = lin.state_dict()
        want_keys = {"packed", "scales"} | ({"bias"} if biases[name] is not None else set())
        assert set(sd) == want_keys
        assert sd["packed"].dtype == torch.int32 and tuple(sd["packed"].shape) == (n, k // 8)
        assert sd["scales"].dtype == torch.float16 and tuple(sd["scales"].shape) == (n, k // group)
        ref_p, ref_s = o.quantize_weight(weights[name].numpy(), group)
        assert np.array_equal(sd["packed"].numpy(), ref_p)
        assert np.array_equal(sd["scales"].numpy().view(np.uint16), ref_s.view(np.uint16))
        if "bias" in sd:
            assert sd["bias"].dtype == torch.float16
            assert torch.equal(sd["bias"], biases[name].detach().half())


def test_state_dict_round_trip():
    torch.manual_seed(4)
    a = KFLinearInt4.from_linear(nn.Linear(256, 128, bias=True), 128)
    b = KFLinearInt4.from_linear(nn.Linear(256, 128, bias=True), 128)
    assert not torch.equal(a.packed, b.packed)
    b.load_state_dict(a.state_dict())
    for key in ("packed", "scales", "bias"):
        assert torch.equal(getattr(a, key), getattr(b, key))


def test_names_select_the_swapped_linears():
    blk = _Block(128, 256, False)
    assert quantize_linears_(blk, 64, names=("gate_proj", "up_proj")) == 2
    assert isinstance(blk.gate_proj, KFLinearInt4) and isinstance(blk.up_proj, KFLinearInt4)
    assert isinstance(blk.q_proj, nn.Linear) and isinstance(blk.down_proj, nn.Linear)


def test_forward_refuses_non_fp16_before_any_launch():
    lin = KFLinearInt4.from_linear(nn.Linear(128, 64, bias=False), 64)
    with pytest.raises(TypeError, match="fp16 activations, got torch.float32"):
        lin(torch.randn(2, 128))
