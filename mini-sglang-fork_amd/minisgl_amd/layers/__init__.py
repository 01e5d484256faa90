from .activation import gelu_and_mul, gelu_and_mul_quant, silu_and_mul, silu_and_mul_quant
from .base import BaseOP, OPList, StateLessOP
from .linear import (
    LinearColParallelMerged,
    LinearOProj,
    LinearQKVMerged,
    LinearReplicated,
    LinearRowParallel,
    quantize_weight,
)
from .mlp import GatedMLPW8A8
from .moe import MoELayer
from .norm import RMSNorm, RMSNormFused, RMSNormQuant

__all__ = [
    "BaseOP",
    "OPList",
    "StateLessOP",
    "LinearColParallelMerged",
    "LinearOProj",
    "LinearQKVMerged",
    "LinearReplicated",
    "LinearRowParallel",
    "quantize_weight",
    "GatedMLPW8A8",
    "MoELayer",
    "RMSNorm",
    "RMSNormFused",
    "RMSNormQuant",
    "silu_and_mul",
    "gelu_and_mul",
    "silu_and_mul_quant",
    "gelu_and_mul_quant",
]
