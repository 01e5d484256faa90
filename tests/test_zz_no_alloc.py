"""The allocation-free GEMM entry point (mw8_gemm_w8a8_bf16_noalloc) against
the workspace entry point (mw8_gemm_w8a8_bf16) through the C ABI: bit-equal
bf16 outputs on two calls in a row, the second with a smaller input, both
through the K split (so the static scratch array carries the int32 partial
tiles), plus a decode-size call without a split; both results also equal
the oracle on a row sample."""

import ctypes

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32
from minisgl_amd.benchmark import linear_case
from minisgl_amd.kernel import quant_per_token, reserve_gemm_workspace
from minisgl_amd.kernel.lib import check, load
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _both(lib, q, s, w, sw, M, N, K):
    st = torch.cuda.current_stream().cuda_stream
    y_ws = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
    y_na = torch.full((M, N), 7.0, dtype=torch.bfloat16, device=DEV)
    ws = reserve_gemm_workspace(torch.device(DEV))
    check(lib.mw8_gemm_w8a8_bf16(q.data_ptr(), s.data_ptr(), w.data_ptr(), sw.data_ptr(), None, y_ws.data_ptr(),
                                 M, N, K, ws.data_ptr(), ws.numel(), ctypes.c_void_p(st)))
    check(lib.mw8_gemm_w8a8_bf16_noalloc(q.data_ptr(), s.data_ptr(), w.data_ptr(), sw.data_ptr(), None,
                                         y_na.data_ptr(), M, N, K, ctypes.c_void_p(st)))
    torch.cuda.synchronize()
    return y_ws, y_na


def test_noalloc_gemm_equals_workspace_gemm():
    lib = load()
    # (M, N, K): down at M=512 (40 tiles of 256x256, each split into 6 K
    # ranges: 60 MiB of partial tiles, nearly the whole scratch), then a
    # smaller input that splits (down at 64 tokens: 40 tiles of 64x128, each
    # split into 6 K ranges), then a decode shape (no split)
    for M, N, K, seed in ((512, 5120, 17408, 1), (64, 5120, 17408, 2), (8, 2048, 1024, 3)):
        announce(f"noalloc gemm M={M} N={N} K={K}")
        c = linear_case(M, K, N, seed=seed)
        q, s = quant_per_token(c["x"].to(DEV))
        w, sw = c["w"].to(DEV), c["s_w"].to(DEV)
        need = lib.mw8_gemm_workspace_bytes(M, N, K)
        if M >= 64:
            assert need > 0, "the case must exercise the K split"
        y_ws, y_na = _both(lib, q, s, w, sw, M, N, K)
        assert torch.equal(y_na.view(torch.int16), y_ws.view(torch.int16)), f"M={M}"
        rows = np.unique(np.r_[0, M - 1, np.linspace(0, M - 1, 12).astype(int)])
        y_ref, *_ = orc.linear_w8a8(f32(c["x"][rows]), c["w"].numpy(), c["s_w"].numpy())
        assert bf16_bits_equal(y_na[torch.as_tensor(rows, device=DEV)], y_ref).all(), f"M={M}"
