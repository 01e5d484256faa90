"""Seeded synthetic inputs of the benchmark configurations.

All tensors are drawn on the CPU from ``torch.Generator().manual_seed(seed)``
so that a CPU checker and the GPU see identical bytes:

* activations: ``x = randn(M, K)``, ``mask = rand(M, K) < 1e-3``,
  ``x[mask] *= 20``, cast to bf16 (0.1 % outliers at 20x);
* weights: ``randint(-127, 128, (N, K), int8)``;
* per-channel scales: ``rand(N) * 9e-3 + 1e-3`` (uniform in [1e-3, 1e-2]).

Draw order for a linear case is x, mask, W, s_w (then bias if any).
"""

from __future__ import annotations

from typing import Dict, List, Tuple

import torch

# Qwen3-14B (hidden 5120, intermediate 17408): (name, K, N)
QWEN3_14B_SHAPES: List[Tuple[str, int, int]] = [
    ("qkv", 5120, 7168),
    ("o_proj", 5120, 5120),
    ("gate_up", 5120, 34816),
    ("down", 17408, 5120),
]
SWEEP_M = [1, 8, 64, 512, 4096, 8192]

# Qwen3-32B decoder-layer GEMM chain at M = 2080: (name, K, N)
QWEN3_32B_CHAIN: List[Tuple[str, int, int]] = [
    ("qkv", 5120, 10240),
    ("o_proj", 8192, 5120),
    ("gate_up", 5120, 51200),
    ("down", 25600, 5120),
]

# One GPU's share of the same layer under tensor parallelism 4 (the
# reference README's Qwen3-32B TP4 serving setup): column-parallel qkv
# (16 q + 2 kv heads of 128) and gate_up shard N, row-parallel o_proj and
# down shard K (each rank quantizes its own K shard; the bf16 partial
# outputs would then be summed by the all-reduce of
# python/minisgl/layers/linear.py:123-127).
QWEN3_32B_TP4_SHARE: List[Tuple[str, int, int]] = [
    ("qkv", 5120, 2560),
    ("o_proj", 2048, 5120),
    ("gate_up", 5120, 12800),
    ("down", 6400, 5120),
]


def activations(M: int, K: int, gen: torch.Generator) -> torch.Tensor:
    x = torch.randn(M, K, generator=gen)
    mask = torch.rand(M, K, generator=gen) < 1e-3
    x[mask] *= 20
    return x.to(torch.bfloat16)


def weights(shape, gen: torch.Generator) -> torch.Tensor:
    return torch.randint(-127, 128, tuple(shape), generator=gen, dtype=torch.int8)


def scales(shape, gen: torch.Generator) -> torch.Tensor:
    return torch.rand(tuple(shape) if not isinstance(shape, int) else (shape,), generator=gen) * 9e-3 + 1e-3


def linear_case(M: int, K: int, N: int, seed: int = 0, bias: bool = False) -> Dict[str, torch.Tensor]:
    gen = torch.Generator().manual_seed(seed)
    out = {
        "x": activations(M, K, gen),
        "w": weights((N, K), gen),
        "s_w": scales(N, gen).float(),
    }
    if bias:
        out["bias"] = torch.randn(N, generator=gen).to(torch.bfloat16)
    return out


def moe_case(
    M: int,
    hidden: int = 2048,
    num_experts: int = 128,
    inter: int = 768,
    seed: int = 0,
) -> Dict[str, torch.Tensor]:
    """Qwen3-30B-A3B-like MoE layer: router logits randn(M, E) as bf16,
    hidden states with the outlier recipe, w1 [E, 2I, H] / w2 [E, H, I] int8
    with per-channel scales."""
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(M, num_experts, generator=gen).to(torch.bfloat16)
    hidden_states = activations(M, hidden, gen)
    w1 = weights((num_experts, 2 * inter, hidden), gen)
    s_w1 = scales((num_experts, 2 * inter), gen).float()
    w2 = weights((num_experts, hidden, inter), gen)
    s_w2 = scales((num_experts, hidden), gen).float()
    return dict(logits=logits, hidden=hidden_states, w1=w1, s_w1=s_w1, w2=w2, s_w2=s_w2)
