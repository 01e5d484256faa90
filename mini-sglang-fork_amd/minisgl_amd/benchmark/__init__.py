from .inputs import (
    QWEN3_14B_SHAPES,
    QWEN3_32B_CHAIN,
    activations,
    linear_case,
    moe_case,
    scales,
    weights,
)
from .perf import perf_hip

__all__ = [
    "QWEN3_14B_SHAPES",
    "QWEN3_32B_CHAIN",
    "activations",
    "linear_case",
    "moe_case",
    "scales",
    "weights",
    "perf_hip",
]
