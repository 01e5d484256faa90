"""Full-output exactness of the large-M dense GEMM at every benchmark shape
with M >= 2080 (the eight Qwen3-14B shapes at M = 4096 / 8192 and the four
Qwen3-32B chain GEMMs at M = 2080), under the tiling the library picks.

The oracle's GEMM is ``acc = q @ W^T`` in exact integers (oracle/w8a8.py
``gemm_i32``); at these sizes its full product is too slow on the CPU, so
the int32 output is pinned through identities of that product that cost
O(MK + NK) on the CPU, each compared exactly in int64:

* every row sum:    ``acc @ 1  == q @ (W^T 1)``
* every column sum: ``1^T acc == (1^T q) @ W^T``
* two Freivalds products ``acc @ r == q @ (W^T r)`` with r uniform in
  [-2^16, 2^16]: a wrong output row escapes one product with probability at
  most 1/(2^17 + 1), and a wrong tile would have to cancel in all four.

Every partial sum stays below 2^63 at these sizes (|acc| <= K * 127^2).
The bf16 output is then compared bit-exactly, element by element, with the
oracle's epilogue applied to the verified accumulators.  The quantized
activations are compared in full with the oracle's quantizer first, and the
expectations are built from the oracle's q.
"""

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32, gemm_identities
from minisgl_amd.benchmark import linear_case
from minisgl_amd.benchmark.inputs import QWEN3_14B_SHAPES, QWEN3_32B_CHAIN
from minisgl_amd.kernel import gemm_w8a8, gemm_w8a8_i32, quant_per_token
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"

SHAPES = [(M, K, N) for M in (4096, 8192) for _, K, N in QWEN3_14B_SHAPES] + [
    (2080, K, N) for _, K, N in QWEN3_32B_CHAIN
]


@pytest.mark.parametrize("M,K,N", SHAPES)
def test_gemm_full_output_exact(M, K, N):
    announce(f"gemm full output M={M} K={K} N={N}")
    c = linear_case(M, K, N, seed=0)
    w_np = c["w"].numpy()
    q_ref, s_ref = orc.quant_per_token(f32(c["x"]))
    q, s_a = quant_per_token(c["x"].to(DEV))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s_a.cpu().numpy(), s_ref)

    w = c["w"].to(DEV)
    acc = gemm_w8a8_i32(q, w)
    y = gemm_w8a8(q, s_a, w, c["s_w"].to(DEV))
    torch.cuda.synchronize()

    gen = np.random.default_rng(M + K + N)
    rs = [gen.integers(-(1 << 16), (1 << 16) + 1, N, dtype=np.int64) for _ in range(2)]
    want_rows, want_cols, want_fr = gemm_identities(q_ref, w_np, rs)

    got_rows = acc.sum(dim=1, dtype=torch.int64).cpu().numpy()
    got_cols = acc.sum(dim=0, dtype=torch.int64).cpu().numpy()
    np.testing.assert_array_equal(got_rows, want_rows, err_msg="row sums")
    np.testing.assert_array_equal(got_cols, want_cols, err_msg="column sums")
    for t, r in enumerate(rs):
        rd = torch.from_numpy(r).to(DEV)
        got = torch.cat([(acc[m0:m0 + 1024].to(torch.int64) * rd).sum(dim=1) for m0 in range(0, M, 1024)])
        np.testing.assert_array_equal(got.cpu().numpy(), want_fr[t], err_msg=f"Freivalds product {t}")

    # bf16: every element against the oracle's epilogue of the verified accumulators
    s_w = c["s_w"].numpy()
    bad = 0
    for m0 in range(0, M, 512):
        a_blk = acc[m0:m0 + 512].cpu().numpy()
        y_ref = orc.epilogue(a_blk, s_ref[m0:m0 + 512], s_w)
        bad += int((~bf16_bits_equal(y[m0:m0 + 512], y_ref)).sum())
    assert bad == 0, f"{bad} of {M * N} bf16 outputs differ"
