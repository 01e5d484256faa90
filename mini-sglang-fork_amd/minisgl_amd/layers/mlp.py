"""W8A8 gated MLP, the caller of the dense path (GatedMLP,
python/minisgl/models/utils.py:25-50): gate_up -> act -> down.  Prefill
batches of GEMM_ACT_MIN_ROWS rows or more apply the activation in the
gate_up GEMM's epilogue (gemm_act_w8a8: no [M, 2I] gate|up tensor) and
quantize the [M, I] activation for the down projection; smaller batches run
the gate_up GEMM and fuse the activation into the requant instead.  Both
paths give the same bits."""

from __future__ import annotations

import torch

from ..kernel import GEMM_ACT_MIN_ROWS, act_and_mul_quant, gemm_act_supported, gemm_act_w8a8, quant_per_token
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
        gu = self.gate_up_proj
        M, K = x.shape[0], x.shape[-1]
        I = gu.weight.shape[0] // 2
        if (M >= GEMM_ACT_MIN_ROWS and x.dim() == 2 and x.is_contiguous() and gu.bias is None
                and gemm_act_supported(M, I, K)):
            q0, s0 = quant_per_token(x)
            act = gemm_act_w8a8(q0, s0, gu.weight, gu.weight_scale, self._act)
            del q0, s0
            q, s = quant_per_token(act)
            del act
        else:
            gate_up = gu.forward(x)
            q, s = act_and_mul_quant(gate_up, self._act)
            del gate_up
        return self.down_proj.forward_quantized(q, s)


__all__ = ["GatedMLPW8A8"]
