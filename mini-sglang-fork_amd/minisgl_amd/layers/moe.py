"""W8A8 MoE layer (mirrors MoELayer, python/minisgl/layers/moe.py:9-59).

Parameters: ``gate_up_proj`` int8 [E, 2I, H] (gate rows first, then up),
``down_proj`` int8 [E, H, I], and their per-output-channel scales
``gate_up_scale`` fp32 [E, 2I] and ``down_scale`` fp32 [E, H].  ``forward``
hands everything to ``ctx.moe_backend`` (:46-56) with the two scales as
extra keyword arguments.  Built at tensor-parallel size 1 (one GPU).
"""

from __future__ import annotations

import torch

from ..core import get_global_ctx
from .base import BaseOP


class MoELayer(BaseOP):
    def __init__(
        self,
        num_experts: int,
        top_k: int,
        hidden_size: int,
        intermediate_size: int,
        renormalize: bool = True,
        activation: str = "silu",
        apply_router_weight_on_input: bool = False,
    ):
        self.num_experts = num_experts
        self.top_k = top_k
        self.hidden_size = hidden_size
        self.intermediate_size = intermediate_size
        self.renormalize = renormalize
        self.activation = activation
        self.apply_router_weight_on_input = apply_router_weight_on_input
        self.gate_up_proj = torch.empty(num_experts, 2 * intermediate_size, hidden_size, dtype=torch.int8)
        self.down_proj = torch.empty(num_experts, hidden_size, intermediate_size, dtype=torch.int8)
        self.gate_up_scale = torch.empty(num_experts, 2 * intermediate_size, dtype=torch.float32)
        self.down_scale = torch.empty(num_experts, hidden_size, dtype=torch.float32)

    def forward(self, hidden_states: torch.Tensor, router_logits: torch.Tensor) -> torch.Tensor:
        ctx = get_global_ctx()
        return ctx.moe_backend.forward(
            hidden_states=hidden_states,
            w1=self.gate_up_proj,
            w2=self.down_proj,
            gating_output=router_logits,
            topk=self.top_k,
            renormalize=self.renormalize,
            activation=self.activation,
            apply_router_weight_on_input=self.apply_router_weight_on_input,
            w1_scale=self.gate_up_scale,
            w2_scale=self.down_scale,
        )


__all__ = ["MoELayer"]
