"""W8A8 checkpoint format and loader (minisgl_amd/checkpoint.py) on the CPU:
a small Qwen3-MoE-style checkpoint is quantized with the oracle, written as
safetensors and streamed back through load_w8a8 -- merges (q|k|v, gate|up),
expert stacking and renamed expert scales, dtype preservation, the
tensor-parallel sharding rules (row-parallel scales replicated), and loading
into the W8A8 layers' state dicts.  GPU checks of quantize_checkpoint are in
test_gpu_checkpoint.py."""

import numpy as np
import pytest
import torch

from minisgl_amd.checkpoint import dummy_w8a8_state, is_quantized_weight, load_w8a8_state_dict, save_w8a8
from minisgl_amd.layers import (
    LinearColParallelMerged,
    LinearOProj,
    LinearQKVMerged,
    LinearRowParallel,
    MoELayer,
    RMSNormFused,
)
from minisgl_amd.layers.base import BaseOP
from oracle import w8a8 as orc

H, NQ, NKV, HD, I, E, IE = 64, 4, 2, 16, 96, 4, 32


def _bf16_checkpoint(seed=0):
    gen = torch.Generator().manual_seed(seed)

    def t(*shape):
        return torch.randn(*shape, generator=gen).to(torch.bfloat16)

    sd = {}
    p0 = "model.layers.0"
    sd[f"{p0}.input_layernorm.weight"] = t(H)
    sd[f"{p0}.self_attn.q_proj.weight"] = t(NQ * HD, H)
    sd[f"{p0}.self_attn.k_proj.weight"] = t(NKV * HD, H)
    sd[f"{p0}.self_attn.v_proj.weight"] = t(NKV * HD, H)
    sd[f"{p0}.self_attn.o_proj.weight"] = t(H, NQ * HD)
    sd[f"{p0}.mlp.gate_proj.weight"] = t(I, H)
    sd[f"{p0}.mlp.up_proj.weight"] = t(I, H)
    sd[f"{p0}.mlp.down_proj.weight"] = t(H, I)
    p1 = "model.layers.1"
    sd[f"{p1}.mlp.gate.weight"] = t(E, H)
    for e in range(E):
        sd[f"{p1}.mlp.experts.{e}.gate_proj.weight"] = t(IE, H)
        sd[f"{p1}.mlp.experts.{e}.up_proj.weight"] = t(IE, H)
        sd[f"{p1}.mlp.experts.{e}.down_proj.weight"] = t(H, IE)
    sd["model.embed_tokens.weight"] = t(50, H)
    return sd


def _oracle_quantize(sd):
    out = {}
    for k, v in sd.items():
        if is_quantized_weight(k):
            q, s = orc.quant_per_token(v.float().numpy())
            out[k] = torch.from_numpy(q)
            out[k.removesuffix(".weight") + ".weight_scale"] = torch.from_numpy(s)
        else:
            out[k] = v
    return out


@pytest.fixture(scope="module")
def ckpt(tmp_path_factory):
    bf = _bf16_checkpoint()
    w8 = _oracle_quantize(bf)
    path = str(tmp_path_factory.mktemp("w8a8") / "model.safetensors")
    save_w8a8(w8, path)
    return bf, w8, path


def test_quantized_key_set():
    assert is_quantized_weight("model.layers.0.self_attn.q_proj.weight")
    assert is_quantized_weight("model.layers.1.mlp.experts.3.down_proj.weight")
    # the MoE router stays bf16 (python/minisgl/models/utils.py:62-66)
    assert not is_quantized_weight("model.layers.1.mlp.gate.weight")
    assert not is_quantized_weight("model.layers.0.input_layernorm.weight")
    assert not is_quantized_weight("model.embed_tokens.weight")
    assert not is_quantized_weight("lm_head.weight")


def test_load_merges_stacks_and_keeps_dtypes(ckpt):
    bf, w8, path = ckpt
    sd = load_w8a8_state_dict(path, num_experts=E)
    p0, p1 = "model.layers.0", "model.layers.1"
    qkv = sd[f"{p0}.self_attn.qkv_proj.weight"]
    assert qkv.dtype == torch.int8 and qkv.shape == ((NQ + 2 * NKV) * HD, H)
    exp = torch.cat([w8[f"{p0}.self_attn.{n}_proj.weight"] for n in "qkv"])
    assert torch.equal(qkv, exp)
    sc = sd[f"{p0}.self_attn.qkv_proj.weight_scale"]
    assert sc.dtype == torch.float32 and torch.equal(sc, torch.cat([w8[f"{p0}.self_attn.{n}_proj.weight_scale"] for n in "qkv"]))
    gu = sd[f"{p0}.mlp.gate_up_proj.weight"]
    assert torch.equal(gu[:I], w8[f"{p0}.mlp.gate_proj.weight"]) and torch.equal(gu[I:], w8[f"{p0}.mlp.up_proj.weight"])
    # experts: packed [E, 2I, H] int8 and [E, 2I] fp32 under the layer's attribute names
    assert sd[f"{p1}.mlp.experts.gate_up_proj"].shape == (E, 2 * IE, H)
    assert sd[f"{p1}.mlp.experts.gate_up_proj"].dtype == torch.int8
    assert sd[f"{p1}.mlp.experts.gate_up_scale"].shape == (E, 2 * IE)
    assert sd[f"{p1}.mlp.experts.down_proj"].shape == (E, H, IE)
    assert sd[f"{p1}.mlp.experts.down_scale"].dtype == torch.float32
    e2 = w8[f"{p1}.mlp.experts.2.up_proj.weight_scale"]
    assert torch.equal(sd[f"{p1}.mlp.experts.gate_up_scale"][2, IE:], e2)
    # non-quantized tensors come back in the model dtype
    assert sd[f"{p0}.input_layernorm.weight"].dtype == torch.bfloat16
    assert torch.equal(sd["model.embed_tokens.weight"], bf["model.embed_tokens.weight"])
    # the values are the oracle's per-channel quantization of the bf16 weight
    q, s = orc.quant_per_token(bf[f"{p0}.mlp.down_proj.weight"].float().numpy())
    np.testing.assert_array_equal(sd[f"{p0}.mlp.down_proj.weight"].numpy(), q)
    np.testing.assert_array_equal(sd[f"{p0}.mlp.down_proj.weight_scale"].numpy(), s)


@pytest.mark.parametrize("rank", [0, 1])
def test_tensor_parallel_sharding_rules(ckpt, rank):
    """tp = 2: column-parallel weights and scales split along dim 0; the k / v
    heads split by head; row-parallel weights split along K with their
    scales replicated; the router and norms replicated."""
    _, w8, path = ckpt
    sd = load_w8a8_state_dict(path, tp_rank=rank, tp_size=2, num_kv_heads=NKV, num_experts=E)
    p0, p1 = "model.layers.0", "model.layers.1"
    q = w8[f"{p0}.self_attn.q_proj.weight"].chunk(2, 0)[rank]
    k = w8[f"{p0}.self_attn.k_proj.weight"].chunk(2, 0)[rank]
    v = w8[f"{p0}.self_attn.v_proj.weight"].chunk(2, 0)[rank]
    assert torch.equal(sd[f"{p0}.self_attn.qkv_proj.weight"], torch.cat([q, k, v]))
    qs = w8[f"{p0}.self_attn.q_proj.weight_scale"].chunk(2, 0)[rank]
    assert torch.equal(sd[f"{p0}.self_attn.qkv_proj.weight_scale"][: qs.numel()], qs)
    o = w8[f"{p0}.self_attn.o_proj.weight"]
    assert torch.equal(sd[f"{p0}.self_attn.o_proj.weight"], o.chunk(2, 1)[rank])
    assert torch.equal(sd[f"{p0}.self_attn.o_proj.weight_scale"], w8[f"{p0}.self_attn.o_proj.weight_scale"])
    assert torch.equal(sd[f"{p0}.mlp.down_proj.weight_scale"], w8[f"{p0}.mlp.down_proj.weight_scale"])
    assert sd[f"{p1}.mlp.experts.down_proj"].shape == (E, H, IE // 2)
    assert sd[f"{p1}.mlp.experts.down_scale"].shape == (E, H)
    assert sd[f"{p1}.mlp.experts.gate_up_scale"].shape == (E, IE)
    assert torch.equal(sd[f"{p1}.mlp.gate.weight"], w8[f"{p1}.mlp.gate.weight"])
    assert sd[f"{p1}.mlp.gate.weight"].dtype == torch.bfloat16  # bf16 router, no weight_scale
    assert f"{p1}.mlp.gate.weight_scale" not in sd


def test_more_tp_ranks_than_kv_heads(ckpt):
    """tp = 4 with 2 kv heads: each rank keeps one whole kv head (two ranks
    per head), as the reference does."""
    _, w8, path = ckpt
    for rank in range(4):
        sd = load_w8a8_state_dict(path, tp_rank=rank, tp_size=4, num_kv_heads=NKV, num_experts=E)
        k = w8["model.layers.0.self_attn.k_proj.weight"]
        head = rank * NKV // 4
        got = sd["model.layers.0.self_attn.qkv_proj.weight"][NQ * HD // 4 : NQ * HD // 4 + HD]
        assert torch.equal(got, k[head * HD : (head + 1) * HD])


class _Block(BaseOP):
    def __init__(self):
        self.input_layernorm = RMSNormFused(H, 1e-6)
        self.qkv_proj = LinearQKVMerged(H, HD, NQ, NKV, has_bias=False)
        self.o_proj = LinearOProj(NQ * HD, H, has_bias=False)
        self.gate_up_proj = LinearColParallelMerged(H, [I, I], has_bias=False)
        self.down_proj = LinearRowParallel(I, H, has_bias=False)
        self.experts = MoELayer(E, 2, H, IE)

    def forward(self):  # pragma: no cover
        raise NotImplementedError


def test_state_dict_loads_into_w8a8_layers(ckpt):
    """The loaded tensors satisfy BaseOP.load_state_dict's shape and dtype
    checks (python/minisgl/layers/base.py:42-46) with no leftover keys."""
    _, _, path = ckpt
    sd = load_w8a8_state_dict(path, num_experts=E)
    p0, p1 = "model.layers.0", "model.layers.1"
    mapped = {
        "input_layernorm.weight": sd[f"{p0}.input_layernorm.weight"],
        "qkv_proj.weight": sd[f"{p0}.self_attn.qkv_proj.weight"],
        "qkv_proj.weight_scale": sd[f"{p0}.self_attn.qkv_proj.weight_scale"],
        "o_proj.weight": sd[f"{p0}.self_attn.o_proj.weight"],
        "o_proj.weight_scale": sd[f"{p0}.self_attn.o_proj.weight_scale"],
        "gate_up_proj.weight": sd[f"{p0}.mlp.gate_up_proj.weight"],
        "gate_up_proj.weight_scale": sd[f"{p0}.mlp.gate_up_proj.weight_scale"],
        "down_proj.weight": sd[f"{p0}.mlp.down_proj.weight"],
        "down_proj.weight_scale": sd[f"{p0}.mlp.down_proj.weight_scale"],
        "experts.gate_up_proj": sd[f"{p1}.mlp.experts.gate_up_proj"],
        "experts.down_proj": sd[f"{p1}.mlp.experts.down_proj"],
        "experts.gate_up_scale": sd[f"{p1}.mlp.experts.gate_up_scale"],
        "experts.down_scale": sd[f"{p1}.mlp.experts.down_scale"],
    }
    blk = _Block()
    blk.load_state_dict(mapped)
    assert blk.qkv_proj.weight.dtype == torch.int8 and blk.experts.down_scale.dtype == torch.float32


def test_dummy_weights_are_valid_int8():
    blk = _Block()
    sd = dummy_w8a8_state(blk.state_dict(), "cpu", seed=3)
    assert sd["qkv_proj.weight"].dtype == torch.int8
    assert int(sd["qkv_proj.weight"].min()) >= -127 and int(sd["qkv_proj.weight"].max()) <= 127
    s = sd["experts.down_scale"]
    assert s.dtype == torch.float32 and float(s.min()) >= 1e-3 and float(s.max()) <= 1e-2
    assert sd["input_layernorm.weight"].dtype == torch.bfloat16
    _Block().load_state_dict(sd)


def test_incomplete_merge_group_is_an_error(tmp_path):
    w8 = _oracle_quantize(_bf16_checkpoint())
    del w8["model.layers.0.self_attn.v_proj.weight"]
    path = str(tmp_path / "broken.safetensors")
    save_w8a8(w8, path)
    with pytest.raises(RuntimeError, match="incomplete merge"):
        load_w8a8_state_dict(path, num_experts=E)
