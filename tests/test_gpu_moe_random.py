"""Seeded random grouped GEMMs (the fused-MoE A10 kernel) through the
default dispatch, checked against the oracle: int32 accumulators and bf16
outputs bit for bit.

Draws the expert count, top-k, token count, alignment block size (16, 32,
64, 128), N and K, and both GEMM roles: gate_up-style (A row = pair //
top_k) and down-style (top_k 1, the routed weight in the epilogue).  The
token counts span the decode ring over gathered rows, the one-tile-per-block
grid and the persistent walk, so the walk's run tables, chunk cuts and
padding skips meet routings the fixed cases do not produce."""

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32
from minisgl_amd.kernel import fused_moe_kernel_w8a8, fused_moe_kernel_w8a8_i32, moe_align_block_size, quant_per_token
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _cases(seed=20261203, count=24):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < count:
        E = int(rng.choice([4, 8, 16, 60, 128, 256]))
        k = int(rng.integers(1, min(8, E) + 1))
        M = int(rng.choice([int(rng.integers(1, 17)), int(rng.integers(17, 257)), int(rng.integers(257, 3001))]))
        B = int(rng.choice([16, 32, 64, 128]))
        N = 16 * int(rng.integers(1, 257))
        K = 16 * int(rng.integers(1, 257))
        which = int(rng.integers(1, 3))
        if M * k * N * K > 2e10:
            continue
        out.append((M, E, k, B, N, K, which))
    return out


@pytest.mark.parametrize("M,E,k,B,N,K,which", _cases())
def test_grouped_gemm_random(M, E, k, B, N, K, which):
    announce(f"grouped random M={M} E={E} k={k} B={B} N={N} K={K} gemm{which}")
    gen = torch.Generator().manual_seed(M * 31 + E * 7 + N + K)
    logits = torch.randn(M, E, generator=gen).to(torch.bfloat16)
    w_ref, ids_ref = orc.topk_softmax(f32(logits), k, True)
    W = torch.randint(-127, 128, (E, N, K), generator=gen, dtype=torch.int8)
    SW = torch.rand(E, N, generator=gen) * 1e-2 + 1e-4
    rows = M if which == 1 else M * k
    act = torch.randn(rows, K, generator=gen).to(torch.bfloat16)
    q, s = quant_per_token(act.to(DEV))
    top_k, routed = (k, None) if which == 1 else (1, w_ref)
    ids, tw = torch.from_numpy(ids_ref).to(DEV), torch.from_numpy(w_ref).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, E)
    Wd, SWd = W.to(DEV), SW.to(DEV)
    out = torch.empty(M * k, N, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(q, s, Wd, SWd, out, tw, sorted_ids, expert_ids, npp, routed is not None, top_k, B, M * k)
    acc = fused_moe_kernel_w8a8_i32(q, Wd, sorted_ids, expert_ids, npp, top_k, B, M * k)
    torch.cuda.synchronize()
    y_ref, acc_ref = orc.grouped_gemm_w8a8(
        q.cpu().numpy(), s.cpu().numpy(), W.numpy(), SW.numpy(), ids_ref, top_k, routed=routed, return_acc=True,
    )
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref)
    eq = bf16_bits_equal(out, y_ref)
    assert eq.all(), f"{(~eq).sum()} of {eq.size} bf16 outputs differ"
