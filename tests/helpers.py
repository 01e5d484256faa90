"""Shared helpers of the parity tests: seeded inputs on the GPU, the CPU
oracle on the same bytes, and comparison utilities."""

from __future__ import annotations

import numpy as np
import torch


def f32(t: torch.Tensor) -> np.ndarray:
    return t.detach().float().cpu().numpy()


def rel_l2(a, b) -> float:
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def bf16_bits_equal(got: torch.Tensor, want_f32: np.ndarray) -> np.ndarray:
    """Elementwise bit equality of a bf16 GPU tensor and bf16-valued fp32 array."""
    g = got.detach().cpu().view(torch.int16).numpy().astype(np.uint16)
    w = (np.ascontiguousarray(want_f32, np.float32).view(np.uint32) >> 16).astype(np.uint16)
    return g == w


def announce(msg: str) -> None:
    print(f"[case] {msg}", flush=True)
