"""nn.Module integration of the INT4 path (reference kernelforge/modules.py:19-65).

- KFLinearInt4: nn.Linear replacement holding packed INT4 weights; forward is ops.int4_linear.
- quantize_linears_: swap a model's decoder linears (q, k, v, o, gate, up, down) for KFLinearInt4.

Inference only.
"""

from __future__ import annotations

import torch
from torch import nn

from kernelforge import ops
from kernelforge import quantize as kq

DECODER_LINEARS = ("q_proj", "k_proj", "v_proj", "o_proj", "gate_proj", "up_proj", "down_proj")


class KFLinearInt4(nn.Module):
    """INT4 weight-only linear: y = x W_hat^T + b, W_hat dequantized inside the HIP kernels.

    Buffers: ``packed`` int32 [N, K/8], ``scales`` fp16 [N, K/G], ``bias`` fp16 [N] or None,
    so ``state_dict()`` carries the packed format.  Activations must be fp16.
    """

    def __init__(self, qw: kq.QuantizedWeight, bias: torch.Tensor | None):
        super().__init__()
        self.out_features, self.in_features = qw.shape
        self.group_size = qw.group_size
        self.register_buffer("packed", qw.packed)
        self.register_buffer("scales", qw.scales)
        self.register_buffer("bias", None if bias is None else bias.detach().half())

    @classmethod
    def from_linear(cls, linear: nn.Linear, group_size: int = kq.DEFAULT_GROUP_SIZE) -> "KFLinearInt4":
        qw = kq.quantize_weight(linear.weight.detach(), group_size)
        return cls(qw, linear.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != torch.float16:
            raise TypeError(f"KFLinearInt4 takes fp16 activations, got {x.dtype}")
        return ops.int4_linear(x, self.packed, self.scales, self.group_size, self.bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"group_size={self.group_size}, int4")


@torch.no_grad()
def quantize_linears_(model: nn.Module, group_size: int = kq.DEFAULT_GROUP_SIZE,
                      names: tuple[str, ...] = DECODER_LINEARS) -> int:
    """Replaces every nn.Linear whose attribute name is in ``names`` with KFLinearInt4, in place.

    Embedding and lm_head stay fp16.  Returns the number of layers replaced.
    """
    found = []
    for parent in model.modules():
        for name, child in parent.named_children():
            if name in names and isinstance(child, nn.Linear):
                found.append((parent, name, child))
    for parent, name, child in found:
        setattr(parent, name, KFLinearInt4.from_linear(child, group_size))
    if torch.cuda.is_available():
        torch.cuda.empty_cache()
    return len(found)
