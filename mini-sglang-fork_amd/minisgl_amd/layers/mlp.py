"""W8A8 gated MLP, the caller of the dense path (GatedMLP,
python/minisgl/models/utils.py:25-50): gate_up -> act -> down, with the
activation fused into the requant of the down projection's input."""

from __future__ import annotations

import torch

from ..kernel import act_and_mul_quant
from .base import BaseOP
from .linear import LinearColParallelMerged, LinearRowParallel


class GatedMLPW8A8(BaseOP):
    def __init__(self, hidden_size: int, intermediate_size: int, hidden_act: str = "silu"):
        if hidden_act not in ("silu", "gelu"):
            raise ValueError(f"Unsupported activation function: {hidden_act}")
        self.gate_up_proj = LinearColParallelMerged(
            hidden_size, [intermediate_size, intermediate_size], has_bias=False
        )
        self.down_proj = LinearRowParallel(intermediate_size, hidden_size, has_bias=False)
        self._act = hidden_act

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate_up = self.gate_up_proj.forward(x)
        q, s = act_and_mul_quant(gate_up, self._act)
        del gate_up
        return self.down_proj.forward_quantized(q, s)


__all__ = ["GatedMLPW8A8"]
