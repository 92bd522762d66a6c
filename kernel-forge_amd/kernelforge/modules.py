"""nn.Module integration of the INT4 path (reference kernelforge/modules.py:19-65).

- KFLinearInt4: nn.Linear replacement holding packed INT4 weights; forward is ops.int4_linear.
- quantize_linears_: swap a model's decoder linears (q, k, v, o, gate, up, down) for KFLinearInt4.
- group_sibling_linears_ (opt-in, no reference counterpart): sibling KFLinearInt4 modules that
  their parent calls on one input (attention's q/k/v, the MLP's gate/up) share one grouped
  launch, behind the module calls the model already makes.

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

    _siblings: "_SiblingLaunch | None" = None
    _slot: int = 0

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if x.dtype != torch.float16:
            raise TypeError(f"KFLinearInt4 takes fp16 activations, got {x.dtype}")
        if self._siblings is not None:
            return self._siblings.output(self._slot, x)
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


# Siblings a decoder calls on one input: Hugging Face's attention (q/k/v on hidden_states) and MLP
# (gate/up on x), and the TinyLlama-architecture model of kernelforge.tinyllama.
SIBLING_GROUPS = (("q_proj", "k_proj", "v_proj"), ("gate_proj", "up_proj"))


class _SiblingLaunch:
    """One ops.int4_linear_grouped call for sibling KFLinearInt4 modules called on the same input.

    The first sibling called on an input launches the group (one GEMV launch at decode sizes, the
    per-problem kernels above them: every output is bit-identical to the sibling's own
    int4_linear) and keeps the other outputs until their modules are called with that same input
    object.  A call with another input while outputs are still waiting - another tensor, or the
    same tensor updated in place since (its version counter moved; tensors made under
    torch.inference_mode() keep no counter, so for them only identity is checked) - means the
    caller does not call the siblings on one input: the waiting outputs are dropped and that call
    runs on its own, so results never depend on the call pattern, only the launch count does.
    Holds references to the input and outputs only until the last sibling has taken its output."""

    def __init__(self, members: list[KFLinearInt4]):
        self.members = members
        self._x: torch.Tensor | None = None
        self._version: int | None = None
        self._ys: list[torch.Tensor] | None = None
        self._pending: set[int] = set()

    @staticmethod
    def _version_of(x: torch.Tensor) -> int | None:
        """x's version counter (bumped by every in-place update), None for inference tensors,
        which keep none."""
        return None if x.is_inference() else x._version

    def output(self, slot: int, x: torch.Tensor) -> torch.Tensor:
        if self._pending:
            if x is self._x and slot in self._pending and self._version_of(x) == self._version:
                y = self._ys[slot]
                self._pending.discard(slot)
                if not self._pending:
                    self._x = self._ys = None
                return y
            self._x, self._ys, self._pending = None, None, set()
            m = self.members[slot]
            return ops.int4_linear(x, m.packed, m.scales, m.group_size, m.bias)
        ms = self.members
        ys = ops.int4_linear_grouped([x] * len(ms), [m.packed for m in ms], [m.scales for m in ms],
                                     ms[0].group_size, [m.bias for m in ms])
        self._x, self._ys, self._pending = x, ys, set(range(len(ms))) - {slot}
        self._version = self._version_of(x)
        return ys[slot]


@torch.no_grad()
def group_sibling_linears_(model: nn.Module, groups: tuple[tuple[str, ...], ...] = SIBLING_GROUPS) -> int:
    """Opt-in: for every module holding all the KFLinearInt4 children named in one of ``groups``
    (same group size and in_features), the parent's calls of those children on one input share a
    single grouped launch (ops.int4_linear_grouped: one GEMV launch at decode sizes instead of one
    per child).  Weights stay in each child's own buffers, in the packed format; state_dict is
    unchanged.  Outputs are bit-identical to the ungrouped modules at every M.  Meant for eager
    and HIP-graph-captured decoding (the pairing is by the identity of the input tensor, which
    torch.compile would specialize on).  Returns the number of groups formed; set a child's
    ``_siblings`` to None to undo."""
    count = 0
    for parent in model.modules():
        for names in groups:
            mods = [getattr(parent, name, None) for name in names]
            if not all(isinstance(m, KFLinearInt4) for m in mods):
                continue
            if len({m.group_size for m in mods}) != 1 or len({m.in_features for m in mods}) != 1:
                continue
            launch = _SiblingLaunch(mods)
            for i, m in enumerate(mods):
                m._siblings, m._slot = launch, i
            count += 1
    return count
