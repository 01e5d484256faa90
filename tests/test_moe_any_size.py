"""CPU tests of the MoE backend's zero padding for hidden and intermediate
sizes that are not multiples of 16 (``padded_experts_w8a8``): the whole
layer computed by the oracle on the padded copies equals, bit for bit, the
oracle on the unpadded problem, and the padded hidden columns come out
zero.  A planted layout mistake (gate and up rows kept adjacent instead of
each half padded on its own) is caught by the same comparison."""

import numpy as np
import pytest
import torch

from minisgl_amd.benchmark import moe_case
from minisgl_amd.moe.fused import padded_experts_w8a8
from oracle import w8a8 as orc


def _f32(t):
    return t.float().numpy()


def _oracle_layer(hidden, w1, s1, w2, s2, logits, k, **kw):
    return orc.fused_moe_w8a8(_f32(hidden), w1.numpy(), s1.numpy(), w2.numpy(), s2.numpy(), _f32(logits), k, **kw)


def _pad_hidden(h, H16):
    hp = torch.zeros(h.shape[0], H16, dtype=h.dtype)
    hp[:, : h.shape[1]] = h
    return hp


@pytest.mark.parametrize(
    "M,E,k,H,I,act,on_input",
    [(5, 8, 2, 100, 40, "silu", False), (12, 6, 3, 72, 8, "gelu", False),
     (9, 4, 2, 48, 20, "silu", True), (7, 5, 2, 30, 32, "silu", False)],
)
def test_padded_layer_equals_unpadded(M, E, k, H, I, act, on_input):
    c = moe_case(M, hidden=H, num_experts=E, inter=I, seed=M + H + I)
    ref = _oracle_layer(c["hidden"], c["w1"], c["s_w1"], c["w2"], c["s_w2"], c["logits"], k,
                        activation=act, apply_router_weight_on_input=on_input)
    w1p, s1p, w2p, s2p = padded_experts_w8a8(c["w1"], c["s_w1"], c["w2"], c["s_w2"])
    H16, I16 = -(-H // 16) * 16, -(-I // 16) * 16
    assert tuple(w1p.shape) == (E, 2 * I16, H16) and tuple(w2p.shape) == (E, H16, I16)
    assert tuple(s1p.shape) == (E, 2 * I16) and tuple(s2p.shape) == (E, H16)
    got = _oracle_layer(_pad_hidden(c["hidden"], H16), w1p, s1p, w2p, s2p, c["logits"], k,
                        activation=act, apply_router_weight_on_input=on_input)
    np.testing.assert_array_equal(orc.bf16_bits(got[:, :H]), orc.bf16_bits(ref))
    assert (got[:, H:] == 0).all()


def test_planted_adjacent_gate_up_is_caught():
    """Padding w1 as one [2I, H] block (gate and up rows adjacent, the zero
    rows after both) puts up rows in the gate half: the layer changes."""
    M, E, k, H, I = 6, 4, 2, 40, 24
    c = moe_case(M, hidden=H, num_experts=E, inter=I, seed=3)
    ref = _oracle_layer(c["hidden"], c["w1"], c["s_w1"], c["w2"], c["s_w2"], c["logits"], k)
    H16, I16 = 48, 32
    w1p = torch.zeros(E, 2 * I16, H16, dtype=torch.int8)
    w1p[:, : 2 * I, :H] = c["w1"]
    s1p = torch.zeros(E, 2 * I16)
    s1p[:, : 2 * I] = c["s_w1"]
    _, _, w2p, s2p = padded_experts_w8a8(c["w1"], c["s_w1"], c["w2"], c["s_w2"])
    got = _oracle_layer(_pad_hidden(c["hidden"], H16), w1p, s1p, w2p, s2p, c["logits"], k)
    assert not np.array_equal(orc.bf16_bits(got[:, :H]), orc.bf16_bits(ref))


def test_padded_copies_are_cached_until_the_weights_change():
    c = moe_case(2, hidden=40, num_experts=4, inter=24, seed=1)
    first = padded_experts_w8a8(c["w1"], c["s_w1"], c["w2"], c["s_w2"])
    assert all(a is b for a, b in zip(first, padded_experts_w8a8(c["w1"], c["s_w1"], c["w2"], c["s_w2"])))
    c["w2"][0, 0, 0] = 7  # an in-place write bumps the version counter
    second = padded_experts_w8a8(c["w1"], c["s_w1"], c["w2"], c["s_w2"])
    assert second[2] is not first[2] and int(second[2][0, 0, 0]) == 7
    s2 = c["s_w2"].clone()  # a new tensor in place of the old one
    third = padded_experts_w8a8(c["w1"], c["s_w1"], c["w2"], s2)
    assert third[3] is not second[3]
