from .lib import MW8Error, load
from .ops import (
    act_and_mul_quant,
    fused_moe_kernel_act_w8a8,
    fused_moe_kernel_w8a8,
    fused_moe_kernel_w8a8_i32,
    gemm_w8a8,
    gemm_w8a8_i32,
    gemm_workspace,
    moe_align_block_size,
    moe_prepare_small,
    moe_sum_reduce,
    quant_per_token,
    rmsnorm_quant,
    topk_softmax,
)

__all__ = [
    "MW8Error",
    "load",
    "act_and_mul_quant",
    "fused_moe_kernel_act_w8a8",
    "fused_moe_kernel_w8a8",
    "fused_moe_kernel_w8a8_i32",
    "gemm_w8a8",
    "gemm_w8a8_i32",
    "gemm_workspace",
    "moe_align_block_size",
    "moe_prepare_small",
    "moe_sum_reduce",
    "quant_per_token",
    "rmsnorm_quant",
    "topk_softmax",
]
