"""RMSNorm layers (python/minisgl/layers/norm.py:8-38) on the fused HIP
kernel, plus the W8A8 variant that hands the next linear its quantized
input directly.

``RMSNorm`` and ``RMSNormFused`` keep the reference's interface (weight
bf16 [size], ``forward`` / ``forward_inplace``; ``RMSNormFused.forward(x,
residual)`` returns ``(normed, residual)`` and works in place when a
residual is given).  ``RMSNormQuant.forward(x, residual)`` returns
``(q, s, residual)``: int8 [M, size] and fp32 [M] ready for a W8A8
linear's ``forward_quantized`` -- norm, residual add and quantization in
one pass over the activations instead of three.

Numerics (one kernel for all three): ``h = x`` or ``bf16(x + residual)``,
``r = 1 / sqrt(fp32(sum h^2 / size) + eps)`` with the sum exact in fp64,
``y = bf16((h * r) * w)``.  The reference's flashinfer kernels are not
available here; their rsqrt and summation order are theirs (the outputs
agree to bf16 rounding).
"""

from __future__ import annotations

from typing import Optional, Tuple

import torch

from ..kernel import rmsnorm_quant
from .base import BaseOP


def _rows(x: torch.Tensor) -> torch.Tensor:
    return x.reshape(-1, x.shape[-1])


class RMSNorm(BaseOP):
    def __init__(self, size: int, eps: float) -> None:
        self.eps = eps
        self.weight = torch.empty(size, dtype=torch.bfloat16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        y = rmsnorm_quant(_rows(x), self.weight, self.eps, quantize=False)
        return y.view_as(x)

    def forward_inplace(self, x: torch.Tensor) -> None:
        x2 = _rows(x)
        rmsnorm_quant(x2, self.weight, self.eps, y=x2, quantize=False)


class RMSNormFused(BaseOP):
    def __init__(self, size: int, eps: float) -> None:
        self.eps = eps
        self.weight = torch.empty(size, dtype=torch.bfloat16)

    def forward(
        self, x: torch.Tensor, residual: Optional[torch.Tensor] = None
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        if residual is None:
            y = rmsnorm_quant(_rows(x), self.weight, self.eps, quantize=False)
            return y.view_as(x), x
        x2 = _rows(x)
        rmsnorm_quant(x2, self.weight, self.eps, residual=_rows(residual), y=x2, quantize=False)
        return x, residual


class RMSNormQuant(BaseOP):
    """RMSNormFused whose output is the int8 input of a W8A8 linear."""

    def __init__(self, size: int, eps: float) -> None:
        self.eps = eps
        self.weight = torch.empty(size, dtype=torch.bfloat16)

    def forward(
        self, x: torch.Tensor, residual: Optional[torch.Tensor] = None
    ) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        x2 = _rows(x)
        if residual is None:
            q, s = rmsnorm_quant(x2, self.weight, self.eps)
            return q, s, x
        q, s = rmsnorm_quant(x2, self.weight, self.eps, residual=_rows(residual))
        return q, s, residual


__all__ = ["RMSNorm", "RMSNormFused", "RMSNormQuant"]
