"""MoE backend plugin interface (python/minisgl/moe/base.py:6-18).  The
W8A8 backend takes two more keyword arguments, ``w1_scale`` and
``w2_scale``, which MoELayer passes."""

from abc import ABC, abstractmethod

import torch


class BaseMoeBackend(ABC):
    @abstractmethod
    def forward(
        self,
        hidden_states: torch.Tensor,
        w1: torch.Tensor,
        w2: torch.Tensor,
        gating_output: torch.Tensor,
        topk: int,
        renormalize: bool,
        activation: str,
        apply_router_weight_on_input: bool,
        **kwargs,
    ) -> torch.Tensor: ...
