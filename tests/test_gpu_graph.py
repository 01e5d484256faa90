"""The drop-ins under HIP graph capture, as the reference engine uses them:
each decode batch size is run eagerly once and then captured
(python/minisgl/engine/graph.py:129-144); a replay reads fresh inputs copied
into the static buffers (:152-158).  Every replay is checked against the
oracle (dense: bit-exact on the replayed inputs; MoE: bit-identical to the
eager layer on the same inputs, and the eager layer against the oracle's
end-to-end chain), with eager work and synchronizations between replays.
No kernel here records a memset, and the dense GEMM's K-split memory is the
library's static per-device scratch, which never moves, so captured pointers
stay valid."""

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32, rel_l2
from minisgl_amd.benchmark.inputs import activations, scales, weights
from minisgl_amd.core import Context, reset_global_ctx, set_global_ctx
from minisgl_amd.kernel import reserve_gemm_workspace
from minisgl_amd.layers import (
    LinearColParallelMerged,
    LinearOProj,
    LinearQKVMerged,
    LinearRowParallel,
    MoELayer,
)
from minisgl_amd.moe import create_moe_backend
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _dense_layers(gen):
    """Qwen3-14B projections: qkv 5120->7168, o 5120->5120, gate_up
    5120->34816, down 17408->5120."""
    layers = {
        "qkv": LinearQKVMerged(5120, 128, 40, 8, has_bias=False),
        "o_proj": LinearOProj(5120, 5120, has_bias=False),
        "gate_up": LinearColParallelMerged(5120, [17408, 17408], has_bias=False),
        "down": LinearRowParallel(17408, 5120, has_bias=False),
    }
    for layer in layers.values():
        N, K = layer.weight.shape
        layer.load_state_dict({"weight": weights((N, K), gen).to(DEV),
                               "weight_scale": scales(N, gen).float().to(DEV)})
    return layers


def _check_dense(layer, x, y, rows):
    ridx = torch.as_tensor(rows, device=DEV)
    y_ref, *_ = orc.linear_w8a8(f32(x[ridx]), layer.weight.cpu().numpy(), layer.weight_scale.cpu().numpy())
    eq = bf16_bits_equal(y[ridx], y_ref)
    assert eq.all(), f"{(~eq).sum()} of {eq.size} bf16 outputs differ"


@pytest.mark.parametrize("bs", [1, 8, 64, 256])
def test_linear_dropins_graph_replay(bs):
    gen = torch.Generator().manual_seed(bs)
    layers = _dense_layers(gen)
    rows = np.arange(bs) if bs <= 8 else np.unique(np.r_[0, bs - 1, np.arange(1, bs - 1, bs // 8)])
    ws_ptr = reserve_gemm_workspace(torch.device(DEV)).data_ptr()
    for name, layer in layers.items():
        announce(f"graph replay {name} bs={bs}")
        K = layer.weight.shape[1]
        x_static = activations(bs, K, gen).to(DEV)
        layer.forward(x_static)  # eager pass before capture, as the engine does
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y_static = layer.forward(x_static)
        for trial in range(3):
            x_new = activations(bs, K, gen).to(DEV)
            x_static.copy_(x_new)
            g.replay()
            # eager work between replays: another shape through the same library
            other = layers["o_proj"].forward(activations(3 * bs + 5, 5120, gen).to(DEV))
            torch.cuda.synchronize()
            _check_dense(layer, x_new, y_static, rows)
            del other
        del g
    assert reserve_gemm_workspace(torch.device(DEV)).data_ptr() == ws_ptr


def test_graphs_survive_later_shapes():
    """Two captures of the o_proj drop-in at M = 40 and M = 100 (tile core
    with a K split through the library's static scratch), then eager calls
    at larger and other sizes (M = 4096, 300, 2080), then both graphs
    replayed on fresh inputs: still bit-exact (the scratch sits at one
    address per device for the life of the process, so no captured pointer
    dangles)."""
    announce("graphs survive later shapes")
    gen = torch.Generator().manual_seed(77)
    layer = _dense_layers(gen)["o_proj"]
    graphs = []
    for M in (40, 100):
        x = activations(M, 5120, gen).to(DEV)
        layer.forward(x)
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = layer.forward(x)
        graphs.append((M, g, x, y))
    for M in (4096, 300, 2080):
        layer.forward(activations(M, 5120, gen).to(DEV))
    torch.cuda.synchronize()
    for M, g, x, y in graphs:
        for _ in range(2):
            x_new = activations(M, 5120, gen).to(DEV)
            x.copy_(x_new)
            g.replay()
            torch.cuda.synchronize()
            _check_dense(layer, x_new, y, np.arange(M))


def _moe_inputs(bs, gen):
    logits = torch.randn(bs, 128, generator=gen).to(torch.bfloat16)
    return activations(bs, 2048, gen), logits


@pytest.mark.parametrize("bs", [1, 8, 16, 64, 256])
def test_moe_layer_graph_replay(bs):
    """MoELayer.forward (config-3 experts: E 128, top-8, H 2048, I 768)
    captured at a decode batch size: the path for the size (up to 16 tokens
    the grouped GEMMs list each expert's pairs from the router ids, GEMM2
    summing the top-k slots; 16-row alignment blocks at 64; 64-row tiles at
    256) replayed on fresh router logits and hidden states."""
    announce(f"moe graph replay bs={bs}")
    gen = torch.Generator().manual_seed(1000 + bs)
    E, H, I = 128, 2048, 768
    w1, s1 = weights((E, 2 * I, H), gen), scales((E, 2 * I), gen).float()
    w2, s2 = weights((E, H, I), gen), scales((E, H), gen).float()
    layer = MoELayer(E, 8, H, I)
    layer.load_state_dict({"gate_up_proj": w1.to(DEV), "down_proj": w2.to(DEV),
                           "gate_up_scale": s1.to(DEV), "down_scale": s2.to(DEV)})
    set_global_ctx(Context(moe_backend=create_moe_backend("fused_w8a8")))
    try:
        h0, lg0 = _moe_inputs(bs, gen)
        h_static, lg_static = h0.to(DEV), lg0.to(DEV)
        layer.forward(h_static.clone(), lg_static)  # eager pass before capture
        torch.cuda.synchronize()
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            out = layer.forward(h_static, lg_static)
        assert out.data_ptr() == h_static.data_ptr()  # in place, like the reference
        for trial in range(2):
            h, lg = _moe_inputs(bs, gen)
            h_static.copy_(h.to(DEV))
            lg_static.copy_(lg.to(DEV))
            g.replay()
            eager = h.to(DEV)
            layer.forward(eager, lg.to(DEV))  # eager work between replays
            torch.cuda.synchronize()
            assert torch.equal(h_static.view(torch.int16), eager.view(torch.int16)), f"trial {trial}"
            ref = orc.fused_moe_w8a8(f32(h), w1.numpy(), s1.numpy(), w2.numpy(), s2.numpy(), f32(lg), 8)
            assert rel_l2(f32(h_static), ref) <= 1e-3, f"trial {trial}"
    finally:
        reset_global_ctx()
