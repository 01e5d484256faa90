"""Seeded random shapes through the default dense dispatch, checked in full
against the oracle: the quantized rows, the int32 accumulators and the bf16
outputs bit for bit (with and without bias).

The fixed-shape tests pin the benchmark shapes and every forced tiling on a
few ragged cases; these draw (M, N, K) across the dispatch regimes -- the
decode core (M <= 32), 33-64 rows (the 64-row ring when K % 128 == 0, else
the decode core), 65-768 rows (the in-block split-K kernel or a ring), and
above (the rings, their K-split tails and the stream walk) -- with N
anywhere from a few columns to past one wave of tiles and K of every
alignment the library takes (16, 64, 128, 256 and 512 bytes), so that tails
of tiles, column ranges, K stages and waves land where the fixed cases do
not put them."""

import numpy as np
import pytest

from helpers import announce
from test_gpu_gemm import _run_case

pytestmark = pytest.mark.gpu


def _shapes(seed=20261202, count=40):
    rng = np.random.default_rng(seed)
    regimes = [(1, 32), (33, 64), (65, 768), (769, 3000)]
    aligns = [16, 64, 128, 256, 512]
    out = []
    while len(out) < count:
        lo, hi = regimes[len(out) % len(regimes)]
        M = int(rng.integers(lo, hi + 1))
        a = aligns[int(rng.integers(0, len(aligns)))]
        K = a * int(rng.integers(1, 8192 // a + 1))
        N = int(rng.integers(1, 12001)) if rng.random() < 0.25 else 8 * int(rng.integers(1, 1501))
        if M * N * K > 4e10:  # keep the CPU oracle to well under a second
            continue
        out.append((M, N, K, bool(rng.random() < 0.3)))
    return out


@pytest.mark.parametrize("M,N,K,bias", _shapes())
def test_gemm_random_shape(M, N, K, bias):
    announce(f"gemm random M={M} N={N} K={K} bias={bias}")
    _run_case(M, K, N, seed=M * 7 + N * 3 + K, bias=bias)


def _wide_shapes(seed=20261204, count=12):
    """Wide N (16384-40000, ragged) at 4-64 tokens with K a multiple of 256:
    the default dispatch's shared-token decode core, with 1-4 token groups
    and 4-12 waves per block."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        M = int(rng.integers(4, 65))
        N = int(rng.integers(16384, 40001))
        K = 256 * int(rng.integers(1, 17))
        if M * N * K > 6e10:
            continue
        out.append((M, N, K, bool(rng.random() < 0.3)))
    return out


@pytest.mark.parametrize("M,N,K,bias", _wide_shapes())
def test_gemm_random_wide_decode(M, N, K, bias):
    from minisgl_amd.kernel.lib import load

    announce(f"gemm random wide M={M} N={N} K={K} bias={bias}")
    assert load().mw8_gemm_kernel_name(M, N, K) == b"decode_sx_gemm_kernel"
    _run_case(M, K, N, seed=M + N + K, bias=bias)
