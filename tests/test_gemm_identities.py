"""CPU checks of the identities that the full-output GPU tests use in place
of the oracle's full product (tests/helpers.py ``gemm_identities``): they
equal the row sums, column sums and Freivalds products of the oracle's
exact ``gemm_i32`` output, and they reject planted mistakes in an output,
including mistakes that cancel in the row sums or in both the row and the
column sums."""

import numpy as np

from helpers import gemm_identities
from oracle import w8a8 as orc


def _sides(acc, rs):
    a = acc.astype(np.int64)
    return a.sum(axis=1), a.sum(axis=0), [a @ r for r in rs]


def _case(seed=0, M=37, K=160, N=9000):
    # N > 4096 exercises the row blocks of the helper
    g = np.random.default_rng(seed)
    q = g.integers(-127, 128, (M, K)).astype(np.int8)
    w = g.integers(-127, 128, (N, K)).astype(np.int8)
    rs = [g.integers(-(1 << 16), (1 << 16) + 1, N, dtype=np.int64) for _ in range(2)]
    return q, w, rs


def _holds(acc, want, rs):
    rows, cols, frs = _sides(acc, rs)
    return (np.array_equal(rows, want[0]), np.array_equal(cols, want[1]),
            all(np.array_equal(f, w) for f, w in zip(frs, want[2])))


def test_identities_equal_the_oracle_product():
    q, w, rs = _case()
    acc = orc.gemm_i32(q, w)
    assert _holds(acc, gemm_identities(q, w, rs), rs) == (True, True, True)


def test_identities_extremes():
    """All +127 activations against all -127 weights: every sum at its bound."""
    M, K, N = 5, 17408, 4100
    q = np.full((M, K), 127, np.int8)
    w = np.full((N, K), -127, np.int8)
    rs = [np.full(N, 1 << 16, np.int64), np.full(N, -(1 << 16), np.int64)]
    acc = np.full((M, N), -K * 127 * 127, np.int64)
    assert _holds(acc, gemm_identities(q, w, rs), rs) == (True, True, True)


def test_identities_reject_planted_mistakes():
    q, w, rs = _case(seed=1)
    want = gemm_identities(q, w, rs)
    acc = orc.gemm_i32(q, w).astype(np.int64)

    one = acc.copy()
    one[3, 4500] += 1  # a single wrong output
    assert _holds(one, want, rs) == (False, False, False)

    pair = acc.copy()  # cancels in its row sum
    pair[7, 10] += 5
    pair[7, 8000] -= 5
    assert _holds(pair, want, rs) == (True, False, False)

    square = acc.copy()  # cancels in the row and the column sums
    square[2, 100] += 3
    square[2, 6000] -= 3
    square[30, 100] -= 3
    square[30, 6000] += 3
    assert _holds(square, want, rs) == (True, True, False)

    swapped = acc.copy()  # two output columns exchanged (a transposed-tile mistake)
    swapped[:, [11, 12]] = swapped[:, [12, 11]]
    rows, cols, frs = _sides(swapped, rs)
    assert np.array_equal(rows, want[0]) and not np.array_equal(cols, want[1])
    assert not any(np.array_equal(f, x) for f, x in zip(frs, want[2]))
