"""The W8A8 MoE layer at hidden and intermediate sizes that are not
multiples of 16 (the backend runs them on zero-padded copies).

For each case: the layer's output (in place, twice, the second call on the
cached padded weights) is bit-identical to the backend run on the same
problem padded by hand; the padded problem's GPU stages are checked against
the oracle on the unpadded problem, stage by stage on the GPU's own stage
inputs (router ids, quantized hidden rows, GEMM1's gate and up halves,
the requant, GEMM2, the slot sum), the padded columns zero throughout; and
the layer equals that staged chain bit for bit.  The cases take every
dispatch path: router-id rows (up to 16 tokens), the one-launch prepare
(over 256 experts), 16-row alignment blocks with GEMM2 and the slot sum
fused, and 64-row prefill blocks with the activation as a separate pass or
in GEMM1's epilogue (K a multiple of 64 after padding), with silu and gelu."""

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from helpers import announce, bf16_bits_equal, f32
from minisgl_amd.benchmark import moe_case
from minisgl_amd.core import Context, reset_global_ctx, set_global_ctx
from minisgl_amd.kernel import (
    act_and_mul_quant,
    fused_moe_kernel_w8a8,
    moe_align_block_size,
    moe_sum_reduce,
    quant_per_token,
    topk_softmax,
)
from minisgl_amd.layers import MoELayer
from minisgl_amd.moe import create_moe_backend
from minisgl_amd.moe.fused import get_default_config
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _up16(n):
    return -(-n // 16) * 16


def _pad_by_hand(c, H, I):
    H16, I16 = _up16(H), _up16(I)
    g, u = c["w1"].split(I, dim=1)
    w1p = torch.cat([F.pad(g, (0, H16 - H, 0, I16 - I)), F.pad(u, (0, H16 - H, 0, I16 - I))], dim=1)
    sg, su = c["s_w1"].split(I, dim=1)
    s1p = torch.cat([F.pad(sg, (0, I16 - I)), F.pad(su, (0, I16 - I))], dim=1)
    w2p = F.pad(c["w2"], (0, I16 - I, 0, H16 - H))
    s2p = F.pad(c["s_w2"], (0, H16 - H))
    hp = F.pad(c["hidden"], (0, H16 - H))
    return [t.to(DEV).contiguous() for t in (hp, w1p, s1p, w2p, s2p)]


@pytest.mark.parametrize(
    "M,E,k,H,I,on_input,act",
    [(1, 8, 2, 100, 40, False, "silu"),      # router-id rows
     (12, 16, 4, 72, 24, True, "silu"),      # router-id rows, routed weight on GEMM1's input
     (5, 300, 2, 40, 8, False, "silu"),      # over 256 experts: router, alignment and quant in one launch
     (40, 64, 2, 200, 56, False, "silu"),    # 16-row blocks, GEMM2 and the slot sum fused
     (300, 8, 2, 136, 40, False, "silu"),    # 64-row blocks, separate activation (H16 = 144)
     (520, 8, 2, 250, 40, True, "silu"),     # 64-row blocks, activation in GEMM1's epilogue (H16 = 256)
     (24, 8, 2, 120, 20, False, "gelu"),     # gelu, 64-row blocks, separate activation
     (600, 8, 2, 250, 24, False, "gelu")],   # gelu in GEMM1's epilogue
)
def test_moe_layer_any_size(M, E, k, H, I, on_input, act):
    announce(f"moe any size M={M} E={E} k={k} H={H} I={I} on_input={on_input} act={act}")
    H16, I16 = _up16(H), _up16(I)
    c = moe_case(M, hidden=H, num_experts=E, inter=I, seed=M + E + H + I)
    layer = MoELayer(E, k, H, I, renormalize=True, activation=act, apply_router_weight_on_input=on_input)
    layer.load_state_dict({
        "gate_up_proj": c["w1"].to(DEV), "down_proj": c["w2"].to(DEV),
        "gate_up_scale": c["s_w1"].to(DEV), "down_scale": c["s_w2"].to(DEV),
    })
    logits = c["logits"].to(DEV)
    hp, w1p, s1p, w2p, s2p = _pad_by_hand(c, H, I)
    set_global_ctx(Context(moe_backend=create_moe_backend("fused_w8a8")))
    try:
        h = c["hidden"].to(DEV)
        out = layer.forward(h, logits)
        out2 = layer.forward(c["hidden"].to(DEV), logits).clone()
        outp = create_moe_backend("fused_w8a8").forward(
            hp.clone(), w1p, w2p, logits, k, True, activation=act, apply_router_weight_on_input=on_input,
            w1_scale=s1p, w2_scale=s2p,
        )
        torch.cuda.synchronize()
    finally:
        reset_global_ctx()
    assert out.data_ptr() == h.data_ptr() and tuple(out.shape) == (M, H)
    assert torch.equal(out.view(torch.int16), outp[:, :H].view(torch.int16))
    assert torch.equal(out2.view(torch.int16), out.view(torch.int16))
    assert not outp[:, H:].any()

    # the padded problem's stages against the oracle on the unpadded problem
    tw, ids = topk_softmax(logits, k, True)
    w_ref, ids_ref = orc.topk_softmax(f32(c["logits"]), k, True)
    np.testing.assert_array_equal(ids.cpu().numpy(), ids_ref)
    hq, hs = quant_per_token(hp)
    q_ref, s_ref = orc.quant_per_token(f32(c["hidden"]))
    np.testing.assert_array_equal(hq[:, :H].cpu().numpy(), q_ref)
    np.testing.assert_array_equal(hs.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    assert not hq[:, H:].any()
    B = get_default_config(M, E, 0, 0, k)["BLOCK_SIZE_M"]
    sorted_ids, expert_ids, npp = moe_align_block_size(ids, B, E)
    routed = tw.cpu().numpy()
    c1 = torch.empty(M * k, 2 * I16, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(hq, hs, w1p, s1p, c1, tw, sorted_ids, expert_ids, npp, on_input, k, B, M * k)
    c1_ref = orc.grouped_gemm_w8a8(q_ref, s_ref, c["w1"].numpy(), c["s_w1"].numpy(), ids_ref, k,
                                   routed=routed if on_input else None)
    assert bf16_bits_equal(c1[:, :I], c1_ref[:, :I]).all()
    assert bf16_bits_equal(c1[:, I16:I16 + I], c1_ref[:, I:]).all()
    assert not c1[:, I:I16].any() and not c1[:, I16 + I:].any()
    qa, sa, a = act_and_mul_quant(c1, act, return_act=True)
    assert not a[:, I:].any()
    qa_ref, sa_ref = orc.quant_per_token(f32(a[:, :I]))
    np.testing.assert_array_equal(qa[:, :I].cpu().numpy(), qa_ref)
    np.testing.assert_array_equal(sa.cpu().numpy().view(np.uint32), sa_ref.view(np.uint32))
    assert not qa[:, I:].any()
    c3 = torch.empty(M * k, H16, dtype=torch.bfloat16, device=DEV)
    fused_moe_kernel_w8a8(qa, sa, w2p, s2p, c3, tw, sorted_ids, expert_ids, npp, not on_input, 1, B, M * k)
    c3_ref = orc.grouped_gemm_w8a8(qa_ref, sa_ref, c["w2"].numpy(), c["s_w2"].numpy(), ids_ref, 1,
                                   routed=None if on_input else routed)
    assert bf16_bits_equal(c3[:, :H], c3_ref).all()
    o = torch.empty(M, H16, dtype=torch.bfloat16, device=DEV)
    moe_sum_reduce(c3.view(M, k, H16), o)
    o_ref = orc.moe_sum_reduce(f32(c3[:, :H]).reshape(M, k, H))
    assert bf16_bits_equal(o[:, :H], o_ref).all()
    assert bf16_bits_equal(out, o_ref).all()  # the layer equals the staged chain
