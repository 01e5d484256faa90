"""quantize_checkpoint on the GPU: the per-channel int8 weights and fp32
scales equal the oracle's quantization bit for bit, the file round-trips
through load_w8a8, and a layer loaded from it computes the W8A8 GEMM."""

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32
from minisgl_amd.checkpoint import load_w8a8_state_dict, quantize_checkpoint, save_w8a8
from minisgl_amd.layers import LinearQKVMerged
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def test_quantize_checkpoint_matches_oracle_and_round_trips(tmp_path):
    announce("quantize_checkpoint")
    gen = torch.Generator().manual_seed(21)
    H, HD, NQ, NKV = 256, 32, 4, 2
    bf = {
        "model.layers.0.self_attn.q_proj.weight": torch.randn(NQ * HD, H, generator=gen).to(torch.bfloat16),
        "model.layers.0.self_attn.k_proj.weight": torch.randn(NKV * HD, H, generator=gen).to(torch.bfloat16),
        "model.layers.0.self_attn.v_proj.weight": torch.randn(NKV * HD, H, generator=gen).to(torch.bfloat16),
        "model.layers.0.input_layernorm.weight": torch.rand(H, generator=gen).to(torch.bfloat16),
    }
    w8 = quantize_checkpoint({k: v.to(DEV) for k, v in bf.items()})
    for n in "qkv":
        key = f"model.layers.0.self_attn.{n}_proj.weight"
        q_ref, s_ref = orc.quant_per_token(f32(bf[key]))
        np.testing.assert_array_equal(w8[key].cpu().numpy(), q_ref)
        np.testing.assert_array_equal(w8[key.replace(".weight", ".weight_scale")].cpu().numpy(), s_ref)
    assert torch.equal(w8["model.layers.0.input_layernorm.weight"].cpu(), bf["model.layers.0.input_layernorm.weight"])
    path = str(tmp_path / "w8a8.safetensors")
    save_w8a8(w8, path)
    sd = load_w8a8_state_dict(path, DEV)
    layer = LinearQKVMerged(H, HD, NQ, NKV, has_bias=False)
    layer.load_state_dict({
        "weight": sd["model.layers.0.self_attn.qkv_proj.weight"],
        "weight_scale": sd["model.layers.0.self_attn.qkv_proj.weight_scale"],
    })
    x = torch.randn(5, H, generator=gen).to(torch.bfloat16)
    y = layer.forward(x.to(DEV))
    y_ref, *_ = orc.linear_w8a8(f32(x), layer.weight.cpu().numpy(), layer.weight_scale.cpu().numpy())
    assert bf16_bits_equal(y, y_ref).all()


def test_quantize_checkpoint_refuses_cpu_tensors():
    with pytest.raises(ValueError, match="GPU"):
        quantize_checkpoint({"a.q_proj.weight": torch.zeros(4, 16, dtype=torch.bfloat16)})
