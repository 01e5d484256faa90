"""The gate_up GEMM with the gated activation in its epilogue
(mw8_gemm_act_w8a8_bf16, GatedMLP.forward's gate_up -> act_fn,
python/minisgl/models/utils.py:44-50).

Its output must equal, bit for bit, the two-step path it replaces: the
plain GEMM into [M, 2I] followed by the activation of act_and_mul_quant
(whose act output is checked against the oracle by the chain and MLP
tests).  Cases: the config-4 gate_up (M = 2080, I = 25600, with the K split
of its short last wave) and its TP-4 share, the Qwen3-14B gate_up at 512
rows, ragged M and I, gelu, and every ring configuration forced through the
tuning override on one ragged shape (tiles past I and past M).  The
requantized activation is checked against the oracle on a row sample."""

import numpy as np
import pytest
import torch

from helpers import announce, f32
from minisgl_amd.benchmark.inputs import activations, scales, weights
from minisgl_amd.kernel import act_and_mul_quant, gemm_act_supported, gemm_act_w8a8, gemm_w8a8, quant_per_token
from minisgl_amd.kernel.lib import load
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _case(M, I, K, seed):
    gen = torch.Generator().manual_seed(seed)
    x = activations(M, K, gen).to(DEV)
    w = weights((2 * I, K), gen).to(DEV)
    sw = scales(2 * I, gen).float().to(DEV)
    q, s = quant_per_token(x)
    return q, s, w, sw


def _two_step(q, s, w, sw, act):
    return act_and_mul_quant(gemm_w8a8(q, s, w, sw), act, return_act=True)[2]


@pytest.mark.parametrize(
    "M,I,K,act",
    [(2080, 25600, 5120, "silu"),   # config 4 gate_up: 9 x 200 tiles, the last 8 split along K
     (2080, 6400, 5120, "silu"),    # its TP-4 share
     (512, 17408, 5120, "silu"),    # Qwen3-14B gate_up at 512 rows
     (300, 1000, 1024, "gelu"),     # ragged M and I
     (129, 264, 256, "silu")],      # a second row tile of one row
)
def test_gemm_act_equals_two_step(M, I, K, act):
    announce(f"gemm_act M={M} I={I} K={K} act={act}")
    assert gemm_act_supported(M, I, K)
    q, s, w, sw = _case(M, I, K, M + I + K)
    got = gemm_act_w8a8(q, s, w, sw, act)
    want = _two_step(q, s, w, sw, act)
    torch.cuda.synchronize()
    assert torch.equal(got.view(torch.int16), want.view(torch.int16))
    # the requant of the fused output against the oracle on a row sample
    rows = np.unique(np.r_[0, M - 1, np.random.default_rng(M).choice(M, 8, replace=False)])
    qa, sa = quant_per_token(got)
    qa_ref, sa_ref = orc.quant_per_token(f32(got[torch.as_tensor(rows, device=DEV)]))
    np.testing.assert_array_equal(qa.cpu().numpy()[rows], qa_ref)
    np.testing.assert_array_equal(sa.cpu().numpy()[rows].view(np.uint32), sa_ref.view(np.uint32))


def test_gemm_act_every_ring_configuration():
    """Every ring configuration the fused activation runs on (and the
    configurations that map to them), forced, on a ragged shape whose last
    tiles run past both I and M; each result equals the two-step path."""
    M, I, K = 333, 1000, 1024
    announce(f"gemm_act forced configurations M={M} I={I} K={K}")
    lib = load()
    q, s, w, sw = _case(M, I, K, 5)
    want = _two_step(q, s, w, sw, "silu")
    try:
        for cfg in range(int(lib.mw8_tuning_count(1))):
            lib.mw8_set_tuning(-1, cfg, -1)
            if not gemm_act_supported(M, I, K):
                continue
            got = gemm_act_w8a8(q, s, w, sw, "silu")
            torch.cuda.synchronize()
            assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"tile cfg {cfg}"
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


def test_gemm_act_rejects_decode_shapes_and_bad_layouts():
    """Decode batches run the plain GEMM (the decode cores), so the fused
    entry declines them; I % 8 != 0 and K % 128 != 0 are declined too."""
    assert not gemm_act_supported(1, 17408, 5120)
    assert not gemm_act_supported(2080, 25604, 5120)
    assert not gemm_act_supported(2080, 25600, 5136)
    assert gemm_act_supported(2080, 25600, 5120)


def test_gated_mlp_takes_the_fused_activation():
    """GatedMLPW8A8.forward at GEMM_ACT_MIN_ROWS rows runs gate_up with the
    activation in its epilogue (no call of the activation + requant kernel)
    and equals the two-step path bit for bit."""
    import minisgl_amd.layers.mlp as mlp_mod
    from minisgl_amd.kernel import GEMM_ACT_MIN_ROWS
    from minisgl_amd.layers import GatedMLPW8A8

    M, H, I = GEMM_ACT_MIN_ROWS, 1024, 2048
    announce(f"gated mlp fused activation M={M}")
    gen = torch.Generator().manual_seed(31)
    mlp = GatedMLPW8A8(H, I)
    for lin in (mlp.gate_up_proj, mlp.down_proj):
        N, K = lin.weight.shape
        lin.load_state_dict({"weight": weights((N, K), gen).to(DEV), "weight_scale": scales(N, gen).float().to(DEV)})
    x = activations(M, H, gen).to(DEV)

    def _no_two_step(*a, **kw):
        raise AssertionError("the fused path called the activation + requant kernel")

    orig = mlp_mod.act_and_mul_quant
    mlp_mod.act_and_mul_quant = _no_two_step
    try:
        out = mlp.forward(x)
    finally:
        mlp_mod.act_and_mul_quant = orig
    q, s = quant_per_token(x)
    qa, sa = act_and_mul_quant(gemm_w8a8(q, s, mlp.gate_up_proj.weight, mlp.gate_up_proj.weight_scale), "silu")
    want = gemm_w8a8(qa, sa, mlp.down_proj.weight, mlp.down_proj.weight_scale)
    torch.cuda.synchronize()
    assert torch.equal(out.view(torch.int16), want.view(torch.int16))
