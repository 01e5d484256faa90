"""GPU parity of the callers of the dense path: the W8A8
gated MLP (GatedMLP.forward, python/minisgl/models/utils.py:44-50) and the
Qwen3-32B decoder-layer GEMM chain of config 4 at M = 2080 (qkv -> o ->
gate_up -> act -> down, the order of python/minisgl/models/qwen3.py:34-41,
attention replaced by the q-slice of the qkv output).

Stage-wise rule: each stage is fed the GPU's own input to that stage; its
int8 quantization, int32 accumulators and bf16 outputs are compared
bit-exactly with the oracle on a row sample (every row of a stage is
independent of the others, so a sample checks whole rows); the activation
itself is held to rel-L2 <= 1e-3.  The drop-in layers' outputs must equal
the staged chain bit for bit."""

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32, rel_l2
from minisgl_amd.benchmark.inputs import activations, scales, weights
from minisgl_amd.kernel import act_and_mul_quant, gemm_w8a8, gemm_w8a8_i32, quant_per_token
from minisgl_amd.layers import GatedMLPW8A8, LinearOProj, LinearQKVMerged
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _load(layer, gen, bias=False):
    N, K = layer.weight.shape
    sd = {"weight": weights((N, K), gen).to(DEV), "weight_scale": scales(N, gen).float().to(DEV)}
    if bias:
        sd["bias"] = torch.randn(N, generator=gen).to(torch.bfloat16).to(DEV)
    layer.load_state_dict(sd)
    return layer


def _rows(M, n, seed):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, M - 1], rng.choice(M, n, replace=False)]))


def _check_quant(x_in, rows):
    """GPU quantization of the stage input, checked on the sampled rows."""
    q, s = quant_per_token(x_in)
    q_ref, s_ref = orc.quant_per_token(f32(x_in[torch.as_tensor(rows, device=DEV)]))
    np.testing.assert_array_equal(q.cpu().numpy()[rows], q_ref)
    np.testing.assert_array_equal(s.cpu().numpy()[rows].view(np.uint32), s_ref.view(np.uint32))
    return q, s, q_ref, s_ref


def _check_gemm(q, s, q_ref, s_ref, layer, rows, what):
    """int32 and bf16 GEMM of one stage on the GPU's own quantized input."""
    w_cpu = layer.weight.cpu().numpy()
    acc = gemm_w8a8_i32(q, layer.weight)
    y = gemm_w8a8(q, s, layer.weight, layer.weight_scale)
    acc_ref = orc.gemm_i32(q_ref, w_cpu)
    np.testing.assert_array_equal(acc.cpu().numpy()[rows], acc_ref, err_msg=f"{what}: int32")
    y_ref = orc.epilogue(acc_ref, s_ref, layer.weight_scale.cpu().numpy())
    ys = y[torch.as_tensor(rows, device=DEV)]
    assert rel_l2(f32(ys), y_ref) <= 1e-3, what
    eq = bf16_bits_equal(ys, y_ref)
    assert eq.all(), f"{what}: {(~eq).sum()} of {eq.size} bf16 outputs differ"
    del acc
    return y


def _chain_stagewise(tag, M, q_heads, kv_heads, inter, seed):
    """One decoder layer's GEMM chain (hidden 5120, heads of 128) at M rows:
    the drop-in layers as a decoder layer calls them, then every stage
    against the oracle on the GPU's own stage input."""
    qc = q_heads * 128
    gen = torch.Generator().manual_seed(seed)
    qkv_proj = _load(LinearQKVMerged(5120, 128, q_heads, kv_heads, has_bias=False), gen)
    o_proj = _load(LinearOProj(qc, 5120, has_bias=False), gen)
    mlp = GatedMLPW8A8(5120, inter)
    _load(mlp.gate_up_proj, gen)
    _load(mlp.down_proj, gen)
    assert qkv_proj.weight.shape == ((q_heads + 2 * kv_heads) * 128, 5120)
    assert mlp.gate_up_proj.weight.shape == (2 * inter, 5120) and mlp.down_proj.weight.shape == (5120, inter)
    x = activations(M, 5120, gen).to(DEV)
    rows = _rows(M, 30, M + seed)

    # the drop-in layers, as a decoder layer calls them
    qkv = qkv_proj.forward(x)
    o = o_proj.forward(qkv[:, :qc])
    out = mlp.forward(o)
    torch.cuda.synchronize()

    # staged, against the oracle
    announce(f"{tag} stage qkv")
    q, s, q_ref, s_ref = _check_quant(x, rows)
    y1 = _check_gemm(q, s, q_ref, s_ref, qkv_proj, rows, "qkv")
    assert torch.equal(y1.view(torch.int16), qkv.view(torch.int16))
    announce(f"{tag} stage o_proj")
    q, s, q_ref, s_ref = _check_quant(y1[:, :qc], rows)
    y2 = _check_gemm(q, s, q_ref, s_ref, o_proj, rows, "o_proj")
    assert torch.equal(y2.view(torch.int16), o.view(torch.int16))
    announce(f"{tag} stage gate_up")
    q, s, q_ref, s_ref = _check_quant(y2, rows)
    y3 = _check_gemm(q, s, q_ref, s_ref, mlp.gate_up_proj, rows, "gate_up")
    announce(f"{tag} stage act + down")
    qa, sa, a = act_and_mul_quant(y3, "silu", return_act=True)
    ridx = torch.as_tensor(rows, device=DEV)
    assert rel_l2(f32(a[ridx]), orc.silu_and_mul(f32(y3[ridx]))) <= 1e-3
    qa_ref, sa_ref = orc.quant_per_token(f32(a[ridx]))
    np.testing.assert_array_equal(qa.cpu().numpy()[rows], qa_ref)
    np.testing.assert_array_equal(sa.cpu().numpy()[rows].view(np.uint32), sa_ref.view(np.uint32))
    del y3, a
    y4 = _check_gemm(qa, sa, qa_ref, sa_ref, mlp.down_proj, rows, "down")
    assert torch.equal(y4.view(torch.int16), out.view(torch.int16))


def test_qwen3_32b_chain_m2080_stagewise():
    """Config 4: hidden 5120, 64 q / 8 kv heads of 128, intermediate 25600,
    M = 2080 (32 decode tokens + a 2048-token prefill chunk as one GEMM
    batch).  GEMM shapes qkv 5120->10240, o 8192->5120, gate_up
    5120->51200, down 25600->5120."""
    announce("cfg4 chain M=2080")
    _chain_stagewise("cfg4", 2080, 64, 8, 25600, 4)


def test_qwen3_32b_tp4_share_m2080_stagewise():
    """One GPU's share of the config-4 layer under tensor parallelism 4 (the
    reference README's Qwen3-32B TP4 setup), at its real shape: 16 q / 2 kv
    heads (qkv 5120->2560), o_proj over the rank's 2048-wide K shard
    (2048->5120), gate_up 5120->12800, down over the 6400-wide K shard
    (6400->5120).  The row-parallel layers quantize their own K shard, which
    is what a rank computes before the all-reduce of the bf16 partials."""
    announce("cfg4 TP4 share chain M=2080")
    _chain_stagewise("cfg4-tp4", 2080, 16, 2, 6400, 44)


@pytest.mark.parametrize("M", [1, 16, 100])
@pytest.mark.parametrize("act", ["silu", "gelu"])
def test_gated_mlp_w8a8(M, act):
    """GatedMLPW8A8.forward at the Qwen3-14B MLP shape (5120 -> 2 x 17408 ->
    5120): gate_up GEMM, fused activation + requant, down GEMM; every stage
    bit-exact against the oracle on the GPU's own stage input (all rows
    for M <= 16, a row sample above), the layer equal to the staged chain."""
    announce(f"gated mlp M={M} act={act}")
    gen = torch.Generator().manual_seed(M + 17)
    mlp = GatedMLPW8A8(5120, 17408, hidden_act=act)
    _load(mlp.gate_up_proj, gen)
    _load(mlp.down_proj, gen)
    x = activations(M, 5120, gen).to(DEV)
    out = mlp.forward(x)
    rows = np.arange(M) if M <= 16 else _rows(M, 14, M)
    q, s, q_ref, s_ref = _check_quant(x, rows)
    gu = _check_gemm(q, s, q_ref, s_ref, mlp.gate_up_proj, rows, "gate_up")
    qa, sa, a = act_and_mul_quant(gu, act, return_act=True)
    ridx = torch.as_tensor(rows, device=DEV)
    want = orc.silu_and_mul(f32(gu[ridx])) if act == "silu" else orc.gelu_and_mul(f32(gu[ridx]))
    assert rel_l2(f32(a[ridx]), want) <= 1e-3
    qa_ref, sa_ref = orc.quant_per_token(f32(a[ridx]))
    np.testing.assert_array_equal(qa.cpu().numpy()[rows], qa_ref)
    y = _check_gemm(qa, sa, qa_ref, sa_ref, mlp.down_proj, rows, "down")
    assert torch.equal(y.view(torch.int16), out.view(torch.int16))


def test_gated_mlp_rejects_unknown_activation():
    with pytest.raises(ValueError):
        GatedMLPW8A8(64, 32, hidden_act="relu")
