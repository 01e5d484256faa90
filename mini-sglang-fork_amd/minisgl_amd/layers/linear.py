"""W8A8 drop-ins for the reference's linear layers
(python/minisgl/layers/linear.py:13-127).

Same constructors and the same ``forward(x: bf16 [..., K]) -> bf16 [..., N]``;
the parameters become ``weight`` int8 [N, K] (the reference's [out, in]
layout, :28), ``weight_scale`` fp32 [N] (per output channel) and ``bias``
bf16 [N] or None.  ``forward`` = per-token int8 quantization of ``x`` +
int8 MFMA GEMM with the scale/bias epilogue, both HIP kernels.

This build runs on one GPU, so every layer is built at tensor-parallel
size 1: local sizes equal full sizes and the row-parallel all-reduce
(:104-105, :125-126) is absent.

Any input size K works, as with ``F.linear``: the GEMM kernels take K in
steps of 16 bytes, so for other K the layer runs the GEMM over the weight
zero-padded to the next multiple of 16 (a copy cached per weight tensor)
and the quantized rows with a zero tail.  Zero columns add nothing to an
int32 dot product, so the output is the unpadded product bit for bit.
"""

from __future__ import annotations

from typing import List, Optional, Tuple

import torch

from ..kernel import gemm_w8a8, linear_bf16_supported, linear_bf16_w8a8, quant_per_token
from .base import BaseOP


def quantize_weight(w: torch.Tensor) -> Tuple[torch.Tensor, torch.Tensor]:
    """Per-output-channel symmetric int8 quantization of a bf16 weight
    [N, K]: ``weight_scale[n] = amax_k |w[n, k]| / 127`` and
    ``weight[n, k] = rint(w[n, k] / weight_scale[n])`` (the same per-row
    kernel as the activation quantizer)."""
    return quant_per_token(w.contiguous())


def _k16(K: int) -> int:
    return (K + 15) // 16 * 16


class _LinearW8A8Impl(BaseOP):
    """Common body of the W8A8 linear layers (mirrors _LinearTPImpl, :13-32)."""

    def __init__(
        self,
        full_isize: int,
        full_osize: int,
        local_isize: int,
        local_osize: int,
        has_bias: bool,
    ):
        self.full_input_size = full_isize
        self.full_output_size = full_osize
        self.local_input_size = local_isize
        self.local_output_size = local_osize
        self.weight = torch.empty(local_osize, local_isize, dtype=torch.int8)
        self.weight_scale = torch.empty(local_osize, dtype=torch.float32)
        self.bias = torch.empty(local_osize, dtype=torch.bfloat16) if has_bias else None

    def forward_quantized(self, q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
        """GEMM + epilogue on an already-quantized input (q int8 [M, K], s fp32 [M])."""
        K = q.shape[1]
        if K % 16 != 0:
            qp = torch.empty((q.shape[0], _k16(K)), dtype=torch.int8, device=q.device)
            qp[:, K:].zero_()
            qp[:, :K].copy_(q)
            return gemm_w8a8(qp, s, self._padded_weight(), self.weight_scale, self.bias)
        return gemm_w8a8(q, s, self.weight, self.weight_scale, self.bias)

    def _padded_weight(self) -> torch.Tensor:
        """``weight`` zero-padded to a multiple of 16 columns, cached per
        weight tensor and version (a new or modified weight rebuilds it)."""
        w = self.weight
        key = (w.data_ptr(), w._version, w.shape)
        if getattr(self, "_wpad_key", None) != key:
            N, K = w.shape
            wp = torch.zeros((N, _k16(K)), dtype=torch.int8, device=w.device)
            wp[:, :K].copy_(w)
            self._wpad, self._wpad_key = wp, key
        return self._wpad

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        lead = x.shape[:-1]
        x2 = x.reshape(-1, x.shape[-1])
        M, K = x2.shape
        N = self.weight.shape[0]
        if (
            0 < M <= 16
            and x2.dtype == torch.bfloat16
            and x2.stride(1) == 1
            and (M == 1 or x2.stride(0) % 8 == 0)
            and x2.data_ptr() % 16 == 0
            and linear_bf16_supported(M, N, K)
        ):
            # decode batch: quantization inside the GEMM launch (one kernel)
            y = linear_bf16_w8a8(x2, self.weight, self.weight_scale, self.bias)
        elif K % 16 != 0:  # quantize into rows with a zero tail up to the GEMM's K step
            qp = torch.empty((M, _k16(K)), dtype=torch.int8, device=x2.device)
            qp[:, K:].zero_()
            _, s = quant_per_token(x2, out=qp[:, :K])
            y = gemm_w8a8(qp, s, self._padded_weight(), self.weight_scale, self.bias)
        else:
            q, s = quant_per_token(x2)
            y = self.forward_quantized(q, s)
        return y.view(*lead, y.shape[-1])

    def load_float_weight(self, w: torch.Tensor, bias: Optional[torch.Tensor] = None) -> None:
        """Quantize a bf16 [N, K] weight on the device into this layer."""
        q, s = quantize_weight(w.to(torch.bfloat16))
        self.weight, self.weight_scale = q, s
        if bias is not None:
            self.bias = bias.to(torch.bfloat16).contiguous()


class LinearReplicated(_LinearW8A8Impl):
    def __init__(self, input_size: int, output_size: int, has_bias: bool):
        super().__init__(input_size, output_size, input_size, output_size, has_bias)


class LinearColParallelMerged(_LinearW8A8Impl):
    """Merged column-parallel layer (gate|up): N = sum(output_sizes) (:56-68)."""

    def __init__(self, input_size: int, output_sizes: List[int], has_bias: bool):
        n = sum(output_sizes)
        super().__init__(input_size, n, input_size, n, has_bias)


class LinearQKVMerged(_LinearW8A8Impl):
    """q|k|v merged: N = (num_qo_heads + 2 * num_kv_heads) * head_dim (:71-88)."""

    def __init__(
        self,
        hidden_size: int,
        head_dim: int,
        num_qo_heads: int,
        num_kv_heads: int,
        has_bias: bool,
    ):
        n = (num_qo_heads + 2 * num_kv_heads) * head_dim
        super().__init__(hidden_size, n, hidden_size, n, has_bias)


class LinearOProj(_LinearW8A8Impl):
    def __init__(self, input_size: int, output_size: int, has_bias: bool):
        super().__init__(input_size, output_size, input_size, output_size, has_bias)


class LinearRowParallel(_LinearW8A8Impl):
    def __init__(self, input_size: int, output_size: int, has_bias: bool):
        super().__init__(input_size, output_size, input_size, output_size, has_bias)


__all__ = [
    "quantize_weight",
    "LinearReplicated",
    "LinearColParallelMerged",
    "LinearQKVMerged",
    "LinearOProj",
    "LinearRowParallel",
]
