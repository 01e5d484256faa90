"""GPU parity of the fused-MoE pieces and the whole W8A8 MoE layer against
the CPU oracle.  Integer outputs (ids, alignment, int8, int32) bit-exact;
bf16 GEMM outputs bit-exact through the closed-form epilogue; router
weights and end-to-end bf16 within rel-L2 1e-3 (stage-wise rule: each stage
is fed the GPU's own input to that stage)."""

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32, rel_l2
from minisgl_amd.benchmark import moe_case
from minisgl_amd.core import Context, reset_global_ctx, set_global_ctx
from minisgl_amd.kernel import (
    act_and_mul_quant,
    fused_moe_kernel_act_w8a8,
    fused_moe_kernel_sum_topk_w8a8,
    fused_moe_kernel_sum_w8a8,
    fused_moe_kernel_topk_w8a8,
    fused_moe_kernel_w8a8,
    fused_moe_kernel_w8a8_i32,
    moe_align_block_size,
    moe_gemm_sum_supported,
    moe_prepare_small,
    moe_route_quant,
    moe_sum_reduce,
    quant_per_token,
    topk_softmax,
    TOPK_ROWS_KERNEL_MAX_TOKENS,
)
from minisgl_amd.layers import MoELayer
from minisgl_amd.moe import create_moe_backend
from minisgl_amd.moe.fused import get_default_config
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_align_docstring_example():
    """Known answer from python/minisgl/moe/fused.py:56-69."""
    announce("align KAT")
    ids = torch.tensor([[2, 3, 4], [1, 2, 4], [1, 3, 4], [1, 2, 3]], dtype=torch.int32, device=DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, 4, 4)
    assert int(npp.item()) == 16
    assert sorted_ids[:16].tolist() == [3, 6, 9, 12, 0, 4, 10, 12, 1, 7, 11, 12, 2, 5, 8, 12]
    assert expert_ids[:4].tolist() == [1, 2, 3, 4]
    assert sorted_ids.numel() == 12 + 5 * 3


@pytest.mark.parametrize("M,B", [(1, 16), (16, 16), (256, 64), (4096, 64), (4096, 16), (300, 128)])
def test_align_matches_oracle(M, B):
    announce(f"align M={M} B={B}")
    c = moe_case(M, seed=M)
    w_ref, ids_ref = orc.topk_softmax(f32(c["logits"]), 8, True)
    ids = torch.from_numpy(ids_ref).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, 128)
    s_ref, e_ref, n_ref = orc.moe_align_block_size(ids_ref, B, 128)
    assert int(npp.item()) == n_ref
    np.testing.assert_array_equal(sorted_ids.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(expert_ids.cpu().numpy()[: n_ref // B], e_ref[: n_ref // B])
    assert (expert_ids.cpu().numpy()[n_ref // B:] == -1).all()


@pytest.mark.parametrize("numel,B,E", [(320000, 64, 128), (8195, 16, 128), (1025, 128, 511), (70001, 64, 7)])
def test_align_large_and_ragged(numel, B, E):
    """Random ids (repeats, a few out of range) over several placement
    blocks, including more than 256K pairs (several pairs per lane)."""
    announce(f"align numel={numel} B={B} E={E}")
    gen = torch.Generator().manual_seed(numel)
    ids = torch.randint(0, E + 1, (numel,), generator=gen, dtype=torch.int32)
    ids[::997] = -1
    ids[5::1999] = E + 7
    sorted_ids, expert_ids, npp = moe_align_block_size(ids.to(DEV), B, E)
    s_ref, e_ref, n_ref = orc.moe_align_block_size(ids.numpy(), B, E)
    assert int(npp.item()) == n_ref
    np.testing.assert_array_equal(sorted_ids.cpu().numpy(), s_ref)
    np.testing.assert_array_equal(expert_ids.cpu().numpy(), e_ref)


@pytest.mark.parametrize("M,E,k,renorm", [(16, 128, 8, True), (256, 128, 8, True), (33, 64, 2, False), (5, 300, 6, True)])
def test_topk_softmax(M, E, k, renorm):
    announce(f"topk M={M} E={E} k={k}")
    gen = torch.Generator().manual_seed(M * E)
    logits = torch.randn(M, E, generator=gen).to(torch.bfloat16)
    w, ids = topk_softmax(logits.to(DEV), k, renorm)
    w_ref, ids_ref = orc.topk_softmax(f32(logits), k, renorm)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    np.testing.assert_allclose(w.cpu().numpy(), w_ref, rtol=2e-6, atol=1e-7)


@pytest.mark.parametrize(
    "M,E,k,renorm,H",
    [(1, 128, 8, True, 2048), (16, 128, 8, True, 2048), (64, 128, 8, True, 2048), (5, 64, 2, False, 40),
     (33, 300, 6, True, 1032), (128, 8, 8, True, 16), (3, 511, 1, False, 5120)],
)
def test_moe_prepare_small_equals_the_separate_kernels(M, E, k, renorm, H):
    """The one-launch decode preparation (router + hidden quantization +
    alignment) against topk_softmax, quant_per_token and
    moe_align_block_size run separately: every output bit-identical (the
    whole sorted_ids / expert_ids buffers included), at the pair bound
    (128 x 8 = 1024), E up to 511 and odd hidden widths."""
    announce(f"moe prepare M={M} E={E} k={k} H={H}")
    gen = torch.Generator().manual_seed(M * 7 + E + k)
    logits = torch.randn(M, E, generator=gen).to(torch.bfloat16).to(DEV)
    hidden = (torch.randn(M, H, generator=gen) * 3).to(torch.bfloat16).to(DEV)
    tw, ids, sorted_ids, expert_ids, npp, q, s = moe_prepare_small(logits, hidden, k, renorm, 16, E)
    tw2, ids2 = topk_softmax(logits, k, renorm)
    q2, s2 = quant_per_token(hidden)
    sorted2, expert2, npp2 = moe_align_block_size(ids2, 16, E)
    torch.cuda.synchronize()
    assert torch.equal(ids, ids2)
    assert torch.equal(tw.view(torch.int32), tw2.view(torch.int32))
    assert torch.equal(q, q2) and torch.equal(s.view(torch.int32), s2.view(torch.int32))
    assert int(npp.item()) == int(npp2.item())
    assert torch.equal(sorted_ids, sorted2) and torch.equal(expert_ids, expert2)
    s_ref, e_ref, n_ref = orc.moe_align_block_size(ids.cpu().numpy(), 16, E)
    assert int(npp.item()) == n_ref
    np.testing.assert_array_equal(sorted_ids.cpu().numpy(), s_ref)


@pytest.mark.parametrize("M,E,k,renorm,H", [(1, 128, 8, True, 2048), (16, 128, 8, True, 2048),
                                            (300, 64, 2, False, 520), (4096, 128, 8, True, 2048),
                                            (37, 300, 6, True, 1024)])
def test_moe_route_quant_equals_the_separate_kernels(M, E, k, renorm, H):
    """Router + hidden quantization in one launch: bit-identical to
    topk_softmax and quant_per_token (which the oracle pins), bf16 logits
    and fp32 logits."""
    announce(f"route+quant M={M} E={E} k={k} H={H}")
    gen = torch.Generator().manual_seed(M + E)
    hid = torch.randn(M, H, generator=gen).to(torch.bfloat16).to(DEV)
    for dt in (torch.bfloat16, torch.float32):
        lg = torch.randn(M, E, generator=gen).to(dt).to(DEV)
        w, ids, q, s = moe_route_quant(lg, hid, k, renorm)
        w_ref, ids_ref = topk_softmax(lg, k, renorm)
        q_ref, s_ref = quant_per_token(hid)
        torch.cuda.synchronize()
        assert torch.equal(ids, ids_ref) and torch.equal(w.view(torch.int32), w_ref.view(torch.int32))
        assert torch.equal(q, q_ref) and torch.equal(s.view(torch.int32), s_ref.view(torch.int32))


def test_moe_prepare_small_rejects_too_many_pairs():
    from minisgl_amd.kernel import MW8Error

    logits = torch.zeros(129, 16, dtype=torch.bfloat16, device=DEV)
    hidden = torch.zeros(129, 64, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(MW8Error):
        moe_prepare_small(logits, hidden, 8, True, 16, 16)


def _grouped(c, M, k, B, which):
    """Run one grouped GEMM on the GPU and on the oracle (same inputs)."""
    w_ref, ids_ref = orc.topk_softmax(f32(c["logits"]), k, True)
    ids = torch.from_numpy(ids_ref).to(DEV)
    tw = torch.from_numpy(w_ref).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, 128)
    if which == 1:
        q, s = quant_per_token(c["hidden"].to(DEV))
        W, SW, top_k, routed = c["w1"], c["s_w1"], k, None
    else:
        gen = torch.Generator().manual_seed(99)
        act = torch.randn(M * k, c["w2"].shape[2], generator=gen).to(torch.bfloat16)
        q, s = quant_per_token(act.to(DEV))
        W, SW, top_k, routed = c["w2"], c["s_w2"], 1, tw
    Wd, SWd = W.to(DEV), SW.to(DEV)
    N = W.shape[1]
    out = torch.empty(M * k, N, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(q, s, Wd, SWd, out, tw, sorted_ids, expert_ids, npp, routed is not None,
                          top_k, B, M * k)
    acc = fused_moe_kernel_w8a8_i32(q, Wd, sorted_ids, expert_ids, npp, top_k, B, M * k)
    torch.cuda.synchronize()
    y_ref, acc_ref = orc.grouped_gemm_w8a8(
        q.cpu().numpy(), s.cpu().numpy(), W.numpy(), SW.numpy(), ids_ref, top_k,
        routed=None if routed is None else w_ref, return_acc=True,
    )
    np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref)
    assert bf16_bits_equal(out, y_ref).all()


@pytest.mark.parametrize("M", [16, 256])
@pytest.mark.parametrize("which", [1, 2])
def test_grouped_gemm(M, which):
    B = get_default_config(M, 128, 0, 0, 8)["BLOCK_SIZE_M"]
    announce(f"grouped gemm{which} M={M} B={B}")
    _grouped(moe_case(M, seed=M), M, 8, B, which)


@pytest.mark.parametrize("B", [16, 32, 128])
def test_grouped_gemm_other_blocks(B):
    announce(f"grouped gemm B={B}")
    _grouped(moe_case(40, seed=40), 40, 8, B, 1)


@pytest.mark.parametrize("which", [1, 2])
def test_grouped_gemm_32_row_blocks(which):
    """32-row alignment blocks (two token groups per ring block) at 256
    tokens: ~16 pairs per expert, experts past 32 pairs span two blocks."""
    announce(f"grouped gemm{which} B=32 M=256")
    _grouped(moe_case(256, seed=7), 256, 8, 32, which)


def _ragged_expert_case(seed, M=50, k=2, E=8, N=208, K=384):
    gen = torch.Generator().manual_seed(seed)
    logits = torch.randn(M, E, generator=gen).to(torch.bfloat16)
    W = torch.randint(-127, 128, (E, N, K), generator=gen, dtype=torch.int8)
    SW = torch.rand(E, N, generator=gen) * 1e-2 + 1e-4
    act = torch.randn(M * k, K, generator=gen).to(torch.bfloat16)
    return logits, W, SW, act


def _tuning_count(kind):
    from minisgl_amd.kernel import lib as mw8lib

    return int(mw8lib.load().mw8_tuning_count(kind))


@pytest.mark.parametrize("shape", ["cfg3", "ragged"])
def test_grouped_every_tile_config(shape):
    """Each grouped tile configuration (forced through mw8_set_tuning) for
    block sizes 64 and 128, gate_up-style (A row = sorted id // top_k, no
    routed weight) and down-style (top_k 1, routed weight), bit-exact
    against one oracle result per case."""
    from minisgl_amd.kernel import lib as mw8lib

    lib = mw8lib.load()
    if shape == "cfg3":
        c = moe_case(96, seed=96)
        M, k = 96, 8
        cases = []
        for which in (1, 2):
            if which == 1:
                act, W, SW = c["hidden"], c["w1"], c["s_w1"]
            else:
                gen = torch.Generator().manual_seed(99)
                act = torch.randn(M * k, c["w2"].shape[2], generator=gen).to(torch.bfloat16)
                W, SW = c["w2"], c["s_w2"]
            cases.append((which, act, W, SW))
        logits = c["logits"]
    else:
        M, k = 50, 2
        logits, W, SW, act = _ragged_expert_case(7, M=M, k=k)
        cases = [(1, act[:M], W, SW), (2, act, W, SW)]
    E = W.shape[0]
    w_ref, ids_ref = orc.topk_softmax(f32(logits), k, True)
    ids = torch.from_numpy(ids_ref).to(DEV)
    tw = torch.from_numpy(w_ref).to(DEV)
    try:
        for which, act, W, SW in cases:
            q, s = quant_per_token(act.to(DEV))
            top_k, routed = (k, None) if which == 1 else (1, tw)
            Wd, SWd = W.to(DEV), SW.to(DEV)
            N = W.shape[1]
            y_ref, acc_ref = orc.grouped_gemm_w8a8(
                q.cpu().numpy(), s.cpu().numpy(), W.numpy(), SW.numpy(), ids_ref, top_k,
                routed=None if routed is None else w_ref, return_acc=True,
            )
            for B in (64, 128):
                sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, E)
                for cfg in range(-1, _tuning_count(2)):
                    announce(f"grouped {shape} gemm{which} B={B} cfg={cfg}")
                    lib.mw8_set_tuning(-1, -1, cfg)
                    out = torch.empty(M * k, N, dtype=torch.bfloat16, device=DEV)
                    fused_moe_kernel_w8a8(q, s, Wd, SWd, out, tw, sorted_ids, expert_ids, npp,
                                          routed is not None, top_k, B, M * k)
                    acc = fused_moe_kernel_w8a8_i32(q, Wd, sorted_ids, expert_ids, npp, top_k, B, M * k)
                    torch.cuda.synchronize()
                    np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref)
                    assert bf16_bits_equal(out, y_ref).all()
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


@pytest.mark.parametrize("shape", ["cfg3", "ragged"])
@pytest.mark.parametrize("B", [64, 128])
def test_fused_activation_gemm_equals_gemm_then_activation(shape, B):
    """GEMM1 with the gated activation in its epilogue against GEMM1 into the
    [pairs, 2I] cache followed by the activation kernel: the [pairs, I]
    activation bit-identical, for silu and gelu, with and without the routed
    weight on the input side.  The ragged case has I = 168 (act tiles of
    128 columns, the second one partial), skewed experts and K = 512."""
    announce(f"fused act gemm {shape} B={B}")
    if shape == "cfg3":
        c = moe_case(512, seed=5)
        M, k, W, SW, hidden, logits = 512, 8, c["w1"], c["s_w1"], c["hidden"], c["logits"]
    else:
        M, k = 700, 2
        logits, W, SW, act_in = _ragged_expert_case(21, M=M, k=k, E=6, N=336, K=512)
        hidden = act_in[:M]
    E, N, K = W.shape
    w_ref, ids_ref = orc.topk_softmax(f32(logits), k, True)
    ids = torch.from_numpy(ids_ref).to(DEV)
    tw = torch.from_numpy(w_ref).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, E)
    q, s = quant_per_token(hidden.to(DEV))
    Wd, SWd = W.to(DEV), SW.to(DEV)
    for act_name in ("silu", "gelu"):
        for routed in (False, True):
            c1 = torch.empty(M * k, N, dtype=torch.bfloat16, device=DEV)
            fused_moe_kernel_w8a8(q, s, Wd, SWd, c1, tw, sorted_ids, expert_ids, npp, routed, k, B, M * k)
            _, _, a_ref = act_and_mul_quant(c1, act_name, return_act=True)
            a = torch.empty(M * k, N // 2, dtype=torch.bfloat16, device=DEV)
            fused_moe_kernel_act_w8a8(q, s, Wd, SWd, a, sorted_ids, expert_ids, npp, k, B, M * k, act_name,
                                      tw if routed else None)
            torch.cuda.synchronize()
            assert torch.equal(a.view(torch.int16), a_ref.view(torch.int16)), f"{act_name} routed={routed}"


@pytest.mark.parametrize("shape", ["cfg3", "ragged", "longk"])
def test_grouped_small_blocks_every_config(shape):
    """16-row alignment blocks (the decode regime) through every small-block
    configuration of the LDS DMA ring with gathered token rows,
    gate_up-style and down-style, bit-exact against the oracle.  The ragged
    case has K and N off the 256 / 16 grids; the long-K case has K = 4160
    (17 ring stages of 256 bytes, split unevenly over the waves)."""
    from minisgl_amd.kernel import lib as mw8lib

    lib = mw8lib.load()
    if shape == "cfg3":
        c = moe_case(16, seed=16)
        M, k = 16, 8
        logits = c["logits"]
        gen = torch.Generator().manual_seed(98)
        act2 = torch.randn(M * k, c["w2"].shape[2], generator=gen).to(torch.bfloat16)
        cases = [(1, c["hidden"], c["w1"], c["s_w1"]), (2, act2, c["w2"], c["s_w2"])]
    elif shape == "ragged":
        M, k = 50, 2
        logits, W, SW, act = _ragged_expert_case(11, M=M, k=k, E=8, N=200, K=336)
        cases = [(1, act[:M], W, SW), (2, act, W, SW)]
    else:
        M, k = 12, 2
        logits, W, SW, act = _ragged_expert_case(12, M=M, k=k, E=6, N=96, K=4160)
        cases = [(1, act[:M], W, SW), (2, act, W, SW)]
    E = cases[0][2].shape[0]
    w_ref, ids_ref = orc.topk_softmax(f32(logits), k, True)
    ids = torch.from_numpy(ids_ref).to(DEV)
    tw = torch.from_numpy(w_ref).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, 16, E)
    try:
        for which, act, W, SW in cases:
            q, s = quant_per_token(act.to(DEV))
            top_k, routed = (k, None) if which == 1 else (1, tw)
            Wd, SWd = W.to(DEV), SW.to(DEV)
            N = W.shape[1]
            y_ref, acc_ref = orc.grouped_gemm_w8a8(
                q.cpu().numpy(), s.cpu().numpy(), W.numpy(), SW.numpy(), ids_ref, top_k,
                routed=None if routed is None else w_ref, return_acc=True,
            )
            for cfg in range(-1, _tuning_count(3)):
                announce(f"grouped small {shape} gemm{which} cfg={cfg}")
                lib.mw8_set_tuning(-1, -1, cfg)
                out = torch.empty(M * k, N, dtype=torch.bfloat16, device=DEV)
                fused_moe_kernel_w8a8(q, s, Wd, SWd, out, tw, sorted_ids, expert_ids, npp,
                                      routed is not None, top_k, 16, M * k)
                acc = fused_moe_kernel_w8a8_i32(q, Wd, sorted_ids, expert_ids, npp, top_k, 16, M * k)
                torch.cuda.synchronize()
                np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref, err_msg=f"cfg {cfg}")
                assert bf16_bits_equal(out, y_ref).all(), f"cfg {cfg}"
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


@pytest.mark.parametrize("B", [64, 128])
def test_grouped_skewed_routing(B):
    """Skewed routing: one expert owns 70 alignment blocks (its run is cut
    into several chunk items), others own 1-3 blocks (short runs), some
    none; N and the pair count are not tile multiples.  Bit-exact int32
    and bf16 for the one-tile-per-block grid and the persistent walk
    (whose item lists cut the long runs into chunks and skip padding
    fragments), gate_up-style (A row = pair // top_k) and down-style
    (top_k 1, routed weight)."""
    from minisgl_amd.kernel import lib as mw8lib

    announce(f"grouped run tiles B={B}")
    lib = mw8lib.load()
    gen = torch.Generator().manual_seed(1234)
    M, k, E, N, K = 4500, 2, 6, 320, 512
    ids = torch.full((M, k), 2, dtype=torch.int32)  # expert 2: 4435 pairs (70 blocks of 64)
    ids[:65, 0] = 0          # expert 0: 65 + 70 pairs
    ids[:65, 1] = 4          # expert 4: 65 pairs (2 blocks of 64)
    ids[65:230, 1] = 5       # expert 5: 165 pairs
    ids[230:300, 1] = 0
    ids[300:, 1] = 3         # expert 3: 4200 pairs; expert 1: none
    perm = torch.randperm(M * k, generator=gen)
    ids = ids.view(-1)[perm].view(M, k).contiguous()
    tw = torch.rand(M, k, generator=gen)
    W = torch.randint(-127, 128, (E, N, K), generator=gen, dtype=torch.int8)
    SW = torch.rand(E, N, generator=gen) * 1e-2 + 1e-4
    ids_ref = ids.numpy()
    idsd, twd, Wd, SWd = ids.to(DEV), tw.to(DEV), W.to(DEV), SW.to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(idsd, B, E)
    try:
        for which in (1, 2):
            rows = M if which == 1 else M * k
            act = torch.randn(rows, K, generator=gen).to(torch.bfloat16)
            q, s = quant_per_token(act.to(DEV))
            top_k, routed = (k, None) if which == 1 else (1, tw.numpy())
            y_ref, acc_ref = orc.grouped_gemm_w8a8(
                q.cpu().numpy(), s.cpu().numpy(), W.numpy(), SW.numpy(), ids_ref, top_k,
                routed=routed, return_acc=True,
            )
            for cfg in range(-1, _tuning_count(2)):
                announce(f"run tiles B={B} gemm{which} cfg={cfg}")
                lib.mw8_set_tuning(-1, -1, cfg)
                out = torch.empty(M * k, N, dtype=torch.bfloat16, device=DEV)
                fused_moe_kernel_w8a8(q, s, Wd, SWd, out, twd, sorted_ids, expert_ids, npp,
                                      routed is not None, top_k, B, M * k)
                acc = fused_moe_kernel_w8a8_i32(q, Wd, sorted_ids, expert_ids, npp, top_k, B, M * k)
                torch.cuda.synchronize()
                np.testing.assert_array_equal(acc.cpu().numpy(), acc_ref, err_msg=f"cfg {cfg}")
                assert bf16_bits_equal(out, y_ref).all(), f"cfg {cfg}"
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


def test_sum_reduce():
    announce("sum reduce")
    gen = torch.Generator().manual_seed(3)
    x = torch.randn(37, 8, 2048, generator=gen).to(torch.bfloat16)
    out = torch.empty(37, 2048, dtype=torch.bfloat16, device=DEV)
    moe_sum_reduce(x.to(DEV), out)
    assert bf16_bits_equal(out, orc.moe_sum_reduce(f32(x))).all()
    # rounding-order case: sequential fp32 gives 0, the exact sum is 1
    y = torch.tensor([[[2.0**24] * 8, [1.0] * 8, [-(2.0**24)] * 8]], dtype=torch.bfloat16)
    o2 = torch.empty(1, 8, dtype=torch.bfloat16, device=DEV)
    moe_sum_reduce(y.to(DEV), o2)
    assert o2.float().abs().max().item() == 0.0


def _gemm2_sum_check(ids_ref, w_ref, W, SW, K, k, routed, seed, invalid=None):
    """Down-projection with the slot sum fused in against (a) the grouped
    GEMM into pair rows followed by moe_sum_reduce on the GPU and (b) the
    oracle's grouped GEMM + slot sum; bit for bit.  ``invalid``: pairs whose
    expert id is E (skipped), which contribute +0 to their token's sum."""
    E, N, _ = W.shape
    P = ids_ref.size
    M = P // k
    gen = torch.Generator().manual_seed(seed)
    act = torch.randn(P, K, generator=gen).to(torch.bfloat16)
    q, s = quant_per_token(act.to(DEV))
    ids = torch.from_numpy(ids_ref.astype(np.int32)).to(DEV)
    tw = torch.from_numpy(w_ref.astype(np.float32)).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, 16, E)
    assert moe_gemm_sum_supported(sorted_ids.shape[0], P, E)
    Wd, SWd = W.to(DEV), SW.to(DEV)
    out = torch.full((M, N), float("nan"), dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_sum_w8a8(q, s, Wd, SWd, out, tw if routed else None, sorted_ids, expert_ids, npp, k, P)
    # oracle: the pairs' rows (zero for skipped pairs), summed in slot order
    ok = ids_ref.reshape(-1) < E
    rows = orc.grouped_gemm_w8a8(q.cpu().numpy(), s.cpu().numpy(), W.numpy(), SW.numpy(),
                                 np.where(ok, ids_ref.reshape(-1), 0), 1,
                                 routed=w_ref.reshape(-1) if routed else None)
    rows[~ok] = 0.0
    ref = orc.moe_sum_reduce(rows.reshape(M, k, N))
    eq = bf16_bits_equal(out, ref)
    assert eq.all(), f"{(~eq).sum()} of {eq.size} outputs differ"
    if invalid is None:  # the two-kernel path writes the same bits
        c3 = torch.empty(P, N, dtype=torch.bfloat16, device=DEV)
        fused_moe_kernel_w8a8(q, s, Wd, SWd, c3, tw, sorted_ids, expert_ids, npp, routed, 1, 16, P)
        o = torch.empty(M, N, dtype=torch.bfloat16, device=DEV)
        moe_sum_reduce(c3.view(M, k, N), o)
        assert torch.equal(out.view(torch.int16), o.view(torch.int16))


@pytest.mark.parametrize("M", [1, 5, 16, 64, 128])
@pytest.mark.parametrize("routed", [True, False])
def test_gemm2_sum_fused_config3(M, routed):
    """Config 3 (E 128, top-8, H 2048, I 768) at decode sizes, routed weight
    in GEMM2 or not (applied on GEMM1's input)."""
    announce(f"gemm2+sum fused M={M} routed={routed}")
    c = moe_case(M, seed=M + 11)
    w_ref, ids_ref = orc.topk_softmax(f32(c["logits"]), 8, True)
    _gemm2_sum_check(ids_ref, w_ref, c["w2"], c["s_w2"], 768, 8, routed, seed=M)


@pytest.mark.parametrize(
    "M,E,k,H,I,on_input",
    [(3, 8, 2, 4096, 1792, False),    # Mixtral-like routing (8 experts, top-2), wide hidden
     (40, 64, 6, 2048, 1408, False),  # DeepSeek-like (64 experts, top-6), I off the 256-byte stage
     (100, 128, 8, 2048, 768, True),  # config 3, routed weight on GEMM1's input
     (7, 256, 8, 1024, 512, False)],  # 256 experts
)
def test_moe_layer_decode_fused_sum_equals_two_kernels(M, E, k, H, I, on_input):
    """Decode batches (M <= E: 16-row blocks) through MoELayer: the layer's
    output with GEMM2 and the slot sum fused is bit-identical to the same
    layer run with GEMM2 into pair rows + moe_sum_reduce (whose stages the
    oracle pins); the all-CPU chain end to end as an informational bound."""
    import minisgl_amd.moe.fused as fused_mod

    announce(f"moe decode fused sum M={M} E={E} k={k} H={H} I={I} on_input={on_input}")
    c = moe_case(M, hidden=H, num_experts=E, inter=I, seed=M + E)
    layer = _moe_layer(c, apply_router_weight_on_input=on_input, E=E, k=k, H=H, I=I)
    set_global_ctx(Context(moe_backend=create_moe_backend("fused_w8a8")))
    outs = []
    orig = fused_mod.moe_gemm_sum_supported
    try:
        for fused_on in (True, False):
            fused_mod.moe_gemm_sum_supported = orig if fused_on else (lambda *a: False)
            h = c["hidden"].to(DEV)
            outs.append(layer.forward(h, c["logits"].to(DEV)).clone())
        torch.cuda.synchronize()
    finally:
        fused_mod.moe_gemm_sum_supported = orig
        reset_global_ctx()
    from minisgl_amd.kernel.lib import load

    assert orig(load().mw8_moe_align_max_padded(M * k, E, 16), M * k, E), "the fused path applies here"
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))
    # end to end against the all-CPU chain: informational beside the bit-identity above (a requant
    # rounding flip between the stages moves a chain, as in test_moe_layer_stagewise)
    ref = orc.fused_moe_w8a8(f32(c["hidden"]), c["w1"].numpy(), c["s_w1"].numpy(), c["w2"].numpy(),
                             c["s_w2"].numpy(), f32(c["logits"]), k, apply_router_weight_on_input=on_input)
    e2e = rel_l2(f32(outs[0]), ref)
    print(f"end-to-end rel-L2 vs CPU chain: {e2e:.3e}")
    assert e2e <= 2e-2


@pytest.mark.parametrize("N,K,E,k,M", [(208, 384, 8, 2, 50), (4096, 256, 4, 4, 33), (24, 1040, 3, 3, 7)])
def test_gemm2_sum_fused_ragged(N, K, E, k, M):
    """Column ranges of 0-1 columns per block (N = 24, 208), more blocks than
    CUs (N = 4096: 8 columns each over 512 blocks), K not a multiple of the
    256-byte stage, skewed routing, and top-k other than 8; then pairs routed
    to expert E (skipped) contribute +0."""
    announce(f"gemm2+sum fused ragged N={N} K={K} E={E} k={k} M={M}")
    gen = torch.Generator().manual_seed(N + K)
    W = torch.randint(-127, 128, (E, N, K), generator=gen, dtype=torch.int8)
    SW = torch.rand(E, N, generator=gen) * 1e-2 + 1e-4
    rng = np.random.default_rng(N)
    ids_ref = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int64)
    ids_ref[: M // 3] = np.minimum(ids_ref[: M // 3], 1)  # skew: a third of the tokens on experts 0-1
    w_ref = rng.random((M, k)).astype(np.float32)
    _gemm2_sum_check(ids_ref, w_ref, W, SW, K, k, True, seed=K)
    bad = ids_ref.copy()
    bad[::4, -1] = E
    _gemm2_sum_check(bad, w_ref, W, SW, K, k, True, seed=K + 1, invalid=True)


def test_moe_gemm_sum_rejects_host_tensors():
    """Every tensor argument of the fused GEMM2 + slot sum is checked for the
    device before any launch: a host (CPU) routed weight, sorted-id list,
    block-expert list or padded count raises ValueError (its host pointer
    never reaches a kernel)."""
    E, N, K, k, M = 8, 64, 256, 2, 4
    P = M * k
    gen = torch.Generator().manual_seed(5)
    ids = torch.randint(0, E, (M, k), generator=gen, dtype=torch.int32)
    q, s = quant_per_token(torch.randn(P, K, generator=gen).to(torch.bfloat16).to(DEV))
    W = torch.randint(-127, 128, (E, N, K), generator=gen, dtype=torch.int8).to(DEV)
    SW = torch.rand(E, N, generator=gen).to(DEV)
    tw = torch.rand(M, k, generator=gen).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids.to(DEV), 16, E)
    out = torch.zeros(M, N, dtype=torch.bfloat16, device=DEV)
    args = dict(topk_weights=tw, sorted_token_ids=sorted_ids, expert_ids=expert_ids, num_tokens_post_padded=npp)
    fused_moe_kernel_sum_w8a8(q, s, W, SW, out, top_k=k, num_valid_tokens=P, **args)
    torch.cuda.synchronize()
    for name in args:
        bad = dict(args, **{name: args[name].cpu()})
        with pytest.raises(ValueError):
            fused_moe_kernel_sum_w8a8(q, s, W, SW, out, top_k=k, num_valid_tokens=P, **bad)
    with pytest.raises(ValueError):
        fused_moe_kernel_topk_w8a8(q[:M], s[:M], W, SW, torch.zeros(P, N, dtype=torch.bfloat16, device=DEV),
                                   ids.to(DEV), tw.cpu())


def _router_id_rows_check(ids_ref, w_ref, E, k, N1, K1, N2, K2, routed_on_input, seed):
    """GEMM1 and GEMM2 + slot sum with each expert's rows listed from the
    router ids, against the same kernels over a 16-row alignment; bit for
    bit.  Pairs routed to an id outside [0, E) are skipped by both (their
    GEMM1 rows are not written; they add +0 to their token's sum)."""
    P = ids_ref.size
    M = P // k
    gen = torch.Generator().manual_seed(seed)
    W1 = torch.randint(-127, 128, (E, N1, K1), generator=gen, dtype=torch.int8).to(DEV)
    S1 = (torch.rand(E, N1, generator=gen) * 1e-2 + 1e-4).to(DEV)
    W2 = torch.randint(-127, 128, (E, N2, K2), generator=gen, dtype=torch.int8).to(DEV)
    S2 = (torch.rand(E, N2, generator=gen) * 1e-2 + 1e-4).to(DEV)
    qh, sh = quant_per_token(torch.randn(M, K1, generator=gen).to(torch.bfloat16).to(DEV))
    qa, sa = quant_per_token(torch.randn(P, K2, generator=gen).to(torch.bfloat16).to(DEV))
    ids = torch.from_numpy(ids_ref.astype(np.int32)).to(DEV)
    tw = torch.from_numpy(w_ref.astype(np.float32)).to(DEV)
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, 16, E)
    valid = torch.from_numpy((ids_ref.reshape(-1) >= 0) & (ids_ref.reshape(-1) < E)).to(DEV)
    # GEMM1 (routed weight on its input when routed_on_input)
    c_ref = torch.zeros(P, N1, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(qh, sh, W1, S1, c_ref, tw, sorted_ids, expert_ids, npp, routed_on_input, k, 16, P)
    c_new = torch.zeros(P, N1, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_topk_w8a8(qh, sh, W1, S1, c_new, ids, tw if routed_on_input else None)
    assert torch.equal(c_new[valid].view(torch.int16), c_ref[valid].view(torch.int16))
    # GEMM2 + slot sum (routed weight here unless it went on GEMM1's input)
    rw = None if routed_on_input else tw
    o_ref = torch.full((M, N2), float("nan"), dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_sum_w8a8(qa, sa, W2, S2, o_ref, rw, sorted_ids, expert_ids, npp, k, P)
    o_new = torch.full((M, N2), float("nan"), dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_sum_topk_w8a8(qa, sa, W2, S2, o_new, ids, rw)
    assert torch.equal(o_new.view(torch.int16), o_ref.view(torch.int16))


@pytest.mark.parametrize(
    "M,E,k,on_input",
    [(1, 128, 8, False), (5, 128, 8, False), (16, 128, 8, True), (16, 8, 2, False), (9, 64, 6, False),
     (16, 256, 8, False), (12, 3, 3, True), (17, 128, 8, False), (32, 128, 8, True), (48, 128, 8, False),
     (40, 8, 2, False), (32, 192, 6, False)],
)
def test_router_id_rows_equal_aligned(M, E, k, on_input):
    """Decode batches (<= 48 tokens, distinct experts per token, units of 16
    pairs per expert): the router-id forms of GEMM1 and of GEMM2 + slot sum
    against the aligned forms, with config-3-like sizes scaled down; then a
    quarter of the pairs routed outside [0, E); then every token routed to
    expert 0 (an expert filling all its units)."""
    announce(f"router-id rows M={M} E={E} k={k} on_input={on_input}")
    rng = np.random.default_rng(M * 1000 + E)
    ids_ref = np.stack([rng.choice(E, k, replace=False) for _ in range(M)]).astype(np.int64)
    w_ref = rng.random((M, k)).astype(np.float32)
    _router_id_rows_check(ids_ref, w_ref, E, k, 384, 1024, 512, 192, on_input, seed=M + E)
    bad = ids_ref.copy()
    bad[::4, 0] = E
    bad[1::4, -1] = -1
    _router_id_rows_check(bad, w_ref, E, k, 384, 1024, 512, 192, on_input, seed=M + E + 1)
    if M in (16, 32, 48):
        full = ids_ref.copy()
        for t in range(M):
            others = [e for e in full[t] if e != 0][: k - 1]
            full[t] = np.array([0] + others)
        assert (full == 0).sum() == M
        _router_id_rows_check(full, w_ref, E, k, 384, 1024, 512, 192, on_input, seed=M + E + 2)


@pytest.mark.parametrize("M", [1, 4, 5, 8, 16, 17, 32, 48])
@pytest.mark.parametrize("on_input", [False, True])
def test_moe_layer_router_id_rows_equal_aligned(M, on_input):
    """MoELayer at config 3 for 1-48 tokens: the router-id rows (no
    alignment launch; the dispatch limit raised to the kernels' limit of 48
    tokens, so that 17-48 tokens take them too) against the same layer
    forced onto the aligned paths (the one-launch preparation up to 4
    tokens, router + alignment above); bit for bit."""
    import minisgl_amd.moe.fused as fused_mod

    announce(f"moe layer router-id rows M={M} on_input={on_input}")
    c = moe_case(M, seed=M + 23)
    layer = _moe_layer(c, apply_router_weight_on_input=on_input)
    set_global_ctx(Context(moe_backend=create_moe_backend("fused_w8a8")))
    outs = []
    orig = fused_mod.TOPK_ROWS_MAX_TOKENS
    try:
        for limit in (TOPK_ROWS_KERNEL_MAX_TOKENS, 0):
            fused_mod.TOPK_ROWS_MAX_TOKENS = limit
            outs.append(layer.forward(c["hidden"].to(DEV), c["logits"].to(DEV)).clone())
        torch.cuda.synchronize()
    finally:
        fused_mod.TOPK_ROWS_MAX_TOKENS = orig
        reset_global_ctx()
    assert torch.equal(outs[0].view(torch.int16), outs[1].view(torch.int16))


@pytest.mark.parametrize("M", [4, 16, 256, 4096])
def test_moe_layer_stagewise(M):
    """Whole W8A8 MoE layer through MoELayer -> ctx.moe_backend ("fused_w8a8"),
    checked stage by stage on the GPU's own intermediate values."""
    announce(f"moe layer M={M}")
    c = moe_case(M, seed=0)
    layer = MoELayer(128, 8, 2048, 768, renormalize=True)
    layer.load_state_dict({
        "gate_up_proj": c["w1"].to(DEV), "down_proj": c["w2"].to(DEV),
        "gate_up_scale": c["s_w1"].to(DEV), "down_scale": c["s_w2"].to(DEV),
    })
    set_global_ctx(Context(moe_backend=create_moe_backend("fused_w8a8")))
    try:
        h = c["hidden"].to(DEV)
        out = layer.forward(h, c["logits"].to(DEV))
        torch.cuda.synchronize()
    finally:
        reset_global_ctx()
    assert out.data_ptr() == h.data_ptr()  # in place, like the reference
    # end-to-end vs the all-CPU chain (informational bound 1e-3 not gated for
    # chains; the stage-wise checks below are the gate)
    ref = orc.fused_moe_w8a8(f32(c["hidden"]), c["w1"].numpy(), c["s_w1"].numpy(),
                             c["w2"].numpy(), c["s_w2"].numpy(), f32(c["logits"]), 8)
    e2e = rel_l2(f32(out), ref)
    print(f"end-to-end rel-L2 vs CPU chain: {e2e:.3e}")
    assert e2e <= 2e-2
    # stage-wise: recompute the GPU stages explicitly and check each one
    logits = c["logits"].to(DEV)
    tw, ids = topk_softmax(logits, 8, True)
    w_ref, ids_ref = orc.topk_softmax(f32(c["logits"]), 8, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    hq, hs = quant_per_token(c["hidden"].to(DEV))
    q_ref, s_ref = orc.quant_per_token(f32(c["hidden"]))
    np.testing.assert_array_equal(hq.cpu().numpy(), q_ref)
    B = get_default_config(M, 128, 0, 0, 8)["BLOCK_SIZE_M"]
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, 128)
    c1 = torch.empty(M * 8, 1536, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(hq, hs, c["w1"].to(DEV), c["s_w1"].to(DEV), c1, tw, sorted_ids,
                          expert_ids, npp, False, 8, B, M * 8)
    c1_ref = orc.grouped_gemm_w8a8(q_ref, s_ref, c["w1"].numpy(), c["s_w1"].numpy(), ids_ref, 8)
    assert bf16_bits_equal(c1, c1_ref).all()
    qa, sa, act = act_and_mul_quant(c1, "silu", return_act=True)
    assert rel_l2(f32(act), orc.silu_and_mul(f32(c1))) <= 1e-3
    qa_ref, sa_ref = orc.quant_per_token(f32(act))
    np.testing.assert_array_equal(qa.cpu().numpy(), qa_ref)
    c3 = torch.empty(M * 8, 2048, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(qa, sa, c["w2"].to(DEV), c["s_w2"].to(DEV), c3, tw, sorted_ids,
                          expert_ids, npp, True, 1, B, M * 8)
    c3_ref = orc.grouped_gemm_w8a8(qa_ref, sa_ref, c["w2"].numpy(), c["s_w2"].numpy(), ids_ref, 1,
                                   routed=tw.cpu().numpy())
    assert bf16_bits_equal(c3, c3_ref).all()
    o = torch.empty(M, 2048, dtype=torch.bfloat16, device=DEV)
    moe_sum_reduce(c3.view(M, 8, 2048), o)
    o_ref = orc.moe_sum_reduce(f32(c3).reshape(M, 8, 2048))
    assert bf16_bits_equal(o, o_ref).all()
    assert bf16_bits_equal(out, o_ref).all()  # the layer's result equals the staged chain


def _moe_layer(c, apply_router_weight_on_input=False, E=128, k=8, H=2048, I=768):
    layer = MoELayer(E, k, H, I, renormalize=True, apply_router_weight_on_input=apply_router_weight_on_input)
    layer.load_state_dict({
        "gate_up_proj": c["w1"].to(DEV), "down_proj": c["w2"].to(DEV),
        "gate_up_scale": c["s_w1"].to(DEV), "down_scale": c["s_w2"].to(DEV),
    })
    return layer


@pytest.mark.parametrize("M", [4, 64, 300, 4096])
def test_moe_layer_router_weight_on_input(M):
    """apply_router_weight_on_input=True through MoELayer: the routed weight
    multiplies GEMM1's epilogue and GEMM2 runs without it
    (python/minisgl/moe/fused.py:201,217).  Stage-wise against the oracle on
    the GPU's own stage inputs, the layer bit-identical to the staged chain,
    and the end-to-end CPU chain within 1e-3."""
    announce(f"moe router weight on input M={M}")
    c = moe_case(M, seed=M + 3)
    layer = _moe_layer(c, apply_router_weight_on_input=True)
    set_global_ctx(Context(moe_backend=create_moe_backend("fused_w8a8")))
    try:
        h = c["hidden"].to(DEV)
        out = layer.forward(h, c["logits"].to(DEV))
        torch.cuda.synchronize()
    finally:
        reset_global_ctx()
    ref = orc.fused_moe_w8a8(f32(c["hidden"]), c["w1"].numpy(), c["s_w1"].numpy(), c["w2"].numpy(),
                             c["s_w2"].numpy(), f32(c["logits"]), 8, apply_router_weight_on_input=True)
    assert rel_l2(f32(out), ref) <= 1e-3
    # stage-wise
    tw, ids = topk_softmax(c["logits"].to(DEV), 8, True)
    w_ref, ids_ref = orc.topk_softmax(f32(c["logits"]), 8, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    hq, hs = quant_per_token(c["hidden"].to(DEV))
    q_ref, s_ref = orc.quant_per_token(f32(c["hidden"]))
    B = get_default_config(M, 128, 0, 0, 8)["BLOCK_SIZE_M"]
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, 128)
    c1 = torch.empty(M * 8, 1536, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(hq, hs, c["w1"].to(DEV), c["s_w1"].to(DEV), c1, tw, sorted_ids, expert_ids, npp,
                          True, 8, B, M * 8)
    c1_ref = orc.grouped_gemm_w8a8(q_ref, s_ref, c["w1"].numpy(), c["s_w1"].numpy(), ids_ref, 8,
                                   routed=tw.cpu().numpy())
    assert bf16_bits_equal(c1, c1_ref).all()
    qa, sa = act_and_mul_quant(c1, "silu")
    _, _, a = act_and_mul_quant(c1, "silu", return_act=True)
    qa_ref, sa_ref = orc.quant_per_token(f32(a))
    np.testing.assert_array_equal(qa.cpu().numpy(), qa_ref)
    c3 = torch.empty(M * 8, 2048, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(qa, sa, c["w2"].to(DEV), c["s_w2"].to(DEV), c3, tw, sorted_ids, expert_ids, npp,
                          False, 1, B, M * 8)
    c3_ref = orc.grouped_gemm_w8a8(qa_ref, sa_ref, c["w2"].numpy(), c["s_w2"].numpy(), ids_ref, 1)
    assert bf16_bits_equal(c3, c3_ref).all()
    o_ref = orc.moe_sum_reduce(f32(c3).reshape(M, 8, 2048))
    assert bf16_bits_equal(out, o_ref).all()


@pytest.mark.parametrize("M", [8, 300])
def test_moe_step_by_step_path(M):
    """The step-by-step orchestration (fused_topk -> fused_experts_impl_w8a8,
    the counterpart of python/minisgl/moe/fused.py:127-227) that the
    backend takes for a non-contiguous router output, bit-identical to the
    fast paths on the same inputs; a non-contiguous hidden_states is
    rejected as the reference rejects it (:142)."""
    from minisgl_amd.moe.fused import fused_experts_impl_w8a8, fused_topk

    announce(f"moe step-by-step M={M}")
    c = moe_case(M, seed=M + 11)
    layer = _moe_layer(c)
    set_global_ctx(Context(moe_backend=create_moe_backend("fused_w8a8")))
    try:
        fast = c["hidden"].to(DEV)
        layer.forward(fast, c["logits"].to(DEV))
        wide = torch.zeros(M, 256, dtype=torch.bfloat16, device=DEV)
        wide[:, :128] = c["logits"].to(DEV)
        slow = c["hidden"].to(DEV)
        layer.forward(slow, wide[:, :128])  # non-contiguous gating_output
        h = c["hidden"].to(DEV)
        tw, ids = fused_topk(h, c["logits"].to(DEV), 8, True)
        direct = fused_experts_impl_w8a8(h, layer.gate_up_proj, layer.gate_up_scale, layer.down_proj,
                                         layer.down_scale, tw, ids)
        torch.cuda.synchronize()
        assert torch.equal(slow.view(torch.int16), fast.view(torch.int16))
        assert torch.equal(direct.view(torch.int16), fast.view(torch.int16))
        strided = torch.zeros(M, 4096, dtype=torch.bfloat16, device=DEV)[:, :2048]
        with pytest.raises(AssertionError, match="contiguous"):
            layer.forward(strided, c["logits"].to(DEV))
    finally:
        reset_global_ctx()
    ref = orc.fused_moe_w8a8(f32(c["hidden"]), c["w1"].numpy(), c["s_w1"].numpy(), c["w2"].numpy(),
                             c["s_w2"].numpy(), f32(c["logits"]), 8)
    assert rel_l2(f32(fast), ref) <= 1e-3


def test_fused_topk_marks_padded_tokens():
    """num_token_non_padded (a device tensor): tokens at or past it get ids
    -1 (python/minisgl/moe/fused.py:25-27), which the alignment skips."""
    from minisgl_amd.moe.fused import fused_topk

    announce("fused_topk padding")
    gen = torch.Generator().manual_seed(9)
    logits = torch.randn(10, 16, generator=gen).to(torch.bfloat16).to(DEV)
    h = torch.zeros(10, 64, dtype=torch.bfloat16, device=DEV)
    w, ids = fused_topk(h, logits, 4, True, num_token_non_padded=torch.tensor(7, device=DEV))
    w_ref, ids_ref = orc.topk_softmax(f32(logits), 4, True)
    got = ids.cpu().numpy()
    np.testing.assert_array_equal(got[:7], ids_ref[:7])
    assert (got[7:] == -1).all()
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, 16, 16)
    torch.cuda.synchronize()
    s = sorted_ids.cpu().numpy()[: int(npp.item())]
    assert set(s[s < 40].tolist()) == set(range(28))  # only the 7 x 4 unpadded pairs are placed


def test_backend_rejects_mismatched_shapes():
    be = create_moe_backend("fused_w8a8")
    h = torch.zeros(2, 40, dtype=torch.bfloat16, device=DEV)
    w2 = torch.zeros(4, 40, 32, dtype=torch.int8, device=DEV)
    for w1 in (torch.zeros(4, 60, 40, dtype=torch.int8, device=DEV),   # 60 rows for I = 32
               torch.zeros(4, 64, 40, dtype=torch.int8, device=DEV)):
        w2x = w2 if w1.shape[1] == 60 else torch.zeros(4, 48, 32, dtype=torch.int8, device=DEV)  # H 48 vs 40
        with pytest.raises(ValueError, match=r"w1 \[E, 2I, H\] and w2 \[E, H, I\]"):
            be.forward(h, w1, w2x, torch.zeros(2, 4, device=DEV), 2, True,
                       w1_scale=torch.ones(4, w1.shape[1], device=DEV),
                       w2_scale=torch.ones(4, w2x.shape[1], device=DEV))
