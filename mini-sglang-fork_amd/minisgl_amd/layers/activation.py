"""Activations of the gated MLP (python/minisgl/layers/activation.py:9-18):
``act(x[:, :d]) * x[:, d:]`` (gate first).  On the W8A8 path the result is
always re-quantized for the next GEMM, so the HIP kernel fuses the two;
``silu_and_mul`` / ``gelu_and_mul`` keep the reference's bf16 signature."""

from __future__ import annotations

import torch

from ..kernel import act_and_mul_quant


def _act_bf16(x: torch.Tensor, activation: str, out: torch.Tensor | None) -> torch.Tensor:
    """The activation alone (no requant): one read of x, one write of the result."""
    x2 = x.reshape(-1, x.shape[-1])
    d = x.shape[-1] // 2
    direct = out is not None and out.is_contiguous()
    a = act_and_mul_quant(x2, activation, quantize=False, act_out=out.view(-1, d) if direct else None)
    if out is not None:
        if not direct:
            out.copy_(a.view(out.shape))
        return out
    return a.view(*x.shape[:-1], d)


def silu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    return _act_bf16(x, "silu", out)


def gelu_and_mul(x: torch.Tensor, out: torch.Tensor | None = None) -> torch.Tensor:
    return _act_bf16(x, "gelu", out)


def silu_and_mul_quant(x: torch.Tensor):
    """Fused ``silu(g) * u`` + per-token int8 requant: (q int8 [R, d], s fp32 [R])."""
    return act_and_mul_quant(x.reshape(-1, x.shape[-1]), "silu")


def gelu_and_mul_quant(x: torch.Tensor):
    return act_and_mul_quant(x.reshape(-1, x.shape[-1]), "gelu")


__all__ = ["silu_and_mul", "gelu_and_mul", "silu_and_mul_quant", "gelu_and_mul_quant"]
