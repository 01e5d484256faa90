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


_BLK_ROWS = 256
_blk_buf = np.empty(0)


def _f64_block(a: np.ndarray, r0: int) -> np.ndarray:
    """Rows [r0, r0 + _BLK_ROWS) of int8 a as float64, in one reused buffer
    (a fresh allocation per block pays its page faults every time)."""
    global _blk_buf
    rows = min(_BLK_ROWS, a.shape[0] - r0)
    if _blk_buf.size < _BLK_ROWS * a.shape[1]:
        _blk_buf = np.empty(_BLK_ROWS * a.shape[1])
    blk = _blk_buf[: rows * a.shape[1]].reshape(rows, a.shape[1])
    blk[...] = a[r0:r0 + rows]
    return blk


def _digits(v: np.ndarray):
    """Balanced base-2^20 digits of int64 v (each in [-2^19, 2^19)), lowest
    first, as float64: v = sum_i d_i 2^(20 i)."""
    v = np.asarray(v, np.int64)
    assert np.abs(v).max(initial=0) < (1 << 60)
    out, rest = [], v.copy()
    while True:
        d = ((rest + (1 << 19)) & ((1 << 20) - 1)) - (1 << 19)
        out.append(d.astype(np.float64))
        rest = (rest - d) >> 20  # exact: rest - d is a multiple of 2^20
        if not rest.any():
            return out


def _combine(parts) -> np.ndarray:
    acc = np.zeros_like(parts[0])
    for p in reversed(parts):
        acc = acc * (1 << 20) + p
    return acc


def _exact_mv(a: np.ndarray, v: np.ndarray) -> np.ndarray:
    """``a @ v`` exactly: a int8 [R, C], v int64 [C] -> int64 [R].  Each digit
    product is a float64 BLAS call whose partial sums stay below
    128 * 2^19 * C < 2^53 (C < 2^26), so it is exact."""
    assert a.shape[1] < (1 << 26)
    ds = _digits(v)
    parts = [np.empty(a.shape[0], np.int64) for _ in ds]
    for r0 in range(0, a.shape[0], _BLK_ROWS):
        blk = _f64_block(a, r0)
        for p, d in zip(parts, ds):
            p[r0:r0 + blk.shape[0]] = np.rint(blk @ d).astype(np.int64)
    return _combine(parts)


def _exact_vm(v: np.ndarray, a: np.ndarray) -> np.ndarray:
    """``v @ a`` exactly: v int64 [R], a int8 [R, C] -> int64 [C] (row blocks
    of _BLK_ROWS keep each float64 partial sum below 128 * 2^19 * 256)."""
    ds = _digits(v)
    parts = [np.zeros(a.shape[1], np.int64) for _ in ds]
    for r0 in range(0, a.shape[0], _BLK_ROWS):
        blk = _f64_block(a, r0)
        for p, d in zip(parts, ds):
            p += np.rint(d[r0:r0 + blk.shape[0]] @ blk).astype(np.int64)
    return _combine(parts)


def gemm_identities(q: np.ndarray, w: np.ndarray, rs) -> tuple:
    """Exact int64 identities of ``acc = q @ w^T`` (q [M, K], w [N, K] int8)
    that cost O(MK + NK): every row sum ``q (w^T 1)``, every column sum
    ``(1^T q) w^T`` and the Freivalds products ``q (w^T r)`` for each r in rs
    (int64 [N])."""
    rows = _exact_mv(q, _exact_vm(np.ones(w.shape[0], np.int64), w))
    cols = _exact_mv(w, _exact_vm(np.ones(q.shape[0], np.int64), q))
    return rows, cols, [_exact_mv(q, _exact_vm(r, w)) for r in rs]
