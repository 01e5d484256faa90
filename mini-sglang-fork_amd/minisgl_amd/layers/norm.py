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

from ..kernel import rmsnorm_quant, rmsnorm_strided
from .base import BaseOP


def _rows(x: torch.Tensor) -> torch.Tensor:
    """x as a contiguous [rows, size] matrix: a view of x when x is
    contiguous, otherwise a copy (which in-place callers copy back)."""
    return x.reshape(-1, x.shape[-1]) if x.is_contiguous() else x.contiguous().view(-1, x.shape[-1])


class RMSNorm(BaseOP):
    def __init__(self, size: int, eps: float) -> None:
        self.eps = eps
        self.weight = torch.empty(size, dtype=torch.bfloat16)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if not x.is_contiguous():
            y = torch.empty(x.shape, dtype=torch.bfloat16, device=x.device)
            if rmsnorm_strided(x, self.weight, self.eps, out=y):
                return y
        y = rmsnorm_quant(_rows(x), self.weight, self.eps, quantize=False)
        return y.view(x.shape)

    def forward_inplace(self, x: torch.Tensor) -> None:
        """Normalizes x in place, also when x is a strided view such as the
        per-head q.view(-1, heads, head_dim) of a qkv split
        (python/minisgl/layers/attention.py:49-53): such views are
        normalized where they lie, and any other layout is normalized in a
        copy that is written back into x."""
        if x.is_contiguous():
            x2 = _rows(x)
            rmsnorm_quant(x2, self.weight, self.eps, y=x2, quantize=False)
        elif not rmsnorm_strided(x, self.weight, self.eps):
            x2 = _rows(x)
            rmsnorm_quant(x2, self.weight, self.eps, y=x2, quantize=False)
            x.copy_(x2.view(x.shape))


class RMSNormFused(BaseOP):
    def __init__(self, size: int, eps: float) -> None:
        self.eps = eps
        self.weight = torch.empty(size, dtype=torch.bfloat16)

    def forward(
        self, x: torch.Tensor, residual: Optional[torch.Tensor] = None
    ) -> Tuple[torch.Tensor, torch.Tensor]:
        if residual is None:
            y = rmsnorm_quant(_rows(x), self.weight, self.eps, quantize=False)
            return y.view(x.shape), x
        # in place on x and residual (fused_add_rmsnorm, python/minisgl/layers/norm.py:33-38);
        # non-contiguous tensors are processed in copies written back afterwards
        x2, r2 = _rows(x), _rows(residual)
        rmsnorm_quant(x2, self.weight, self.eps, residual=r2, y=x2, quantize=False)
        if not x.is_contiguous():
            x.copy_(x2.view(x.shape))
        if not residual.is_contiguous():
            residual.copy_(r2.view(residual.shape))
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
        r2 = _rows(residual)
        q, s = rmsnorm_quant(x2, self.weight, self.eps, residual=r2)
        if not residual.is_contiguous():
            residual.copy_(r2.view(residual.shape))
        return q, s, residual


__all__ = ["RMSNorm", "RMSNormFused", "RMSNormQuant"]
