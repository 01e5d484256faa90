"""GPU parity of the per-token quantizer and the fused activation + requant
(HIP kernels via the C ABI) against the CPU oracle: int8 and scales
bit-exact, bf16 activations within rel-L2 1e-3."""

import numpy as np
import pytest
import torch

from helpers import announce, f32, rel_l2
from minisgl_amd.benchmark import activations
from minisgl_amd.kernel import MW8Error, act_and_mul_quant, quant_per_token
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _check_quant(x_bf16: torch.Tensor):
    q, s = quant_per_token(x_bf16.to(DEV))
    torch.cuda.synchronize()
    q_ref, s_ref = orc.quant_per_token(f32(x_bf16))
    np.testing.assert_array_equal(s.cpu().numpy().view(np.uint32), s_ref.view(np.uint32))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)


@pytest.mark.parametrize(
    "M,K",
    [(1, 1024), (1, 5120), (3, 8), (16, 1024), (64, 1024), (33, 5120), (5, 17408),
     (7, 25600), (2, 32768), (3, 40000), (4, 1004), (129, 2048), (1000, 768),
     # every (threads per row, vectors per thread) class of the row kernels
     (2, 1280), (3, 3072), (5, 4104), (2, 6144), (2, 12288), (3, 8200),
     # two rows per wave (32 threads per row): odd row counts leave half a wave idle
     (37, 768), (5, 256), (9, 552), (4097, 768)],
)
def test_quant_seeded_bitexact(M, K):
    announce(f"quant M={M} K={K}")
    gen = torch.Generator().manual_seed(M * 131 + K)
    _check_quant(activations(M, K, gen))


def test_quant_hand_rows():
    announce("quant hand rows")
    rows = np.zeros((6, 16), np.float32)
    rows[0, :6] = [127.0, 2.5, -0.5, 126.5, 3.5, -1.5]  # s == 1: exact ties -> even
    rows[1, 3] = -3.0  # single value -> -127
    rows[3, :4] = [20.0, -0.078125, 0.15625, 1e-3]  # outlier row
    rows[4, :3] = [2.0**-130, -(2.0**-133), 2.0**-128]  # bf16 subnormal row
    rows[5, :4] = [1.0, 1.0 / 254.0, 3.0 / 254.0, -5.0 / 254.0]  # ties at s = 1/127
    x = torch.from_numpy(orc.bf16_round(rows)).to(torch.bfloat16)
    _check_quant(x)
    q, s = quant_per_token(x.to(DEV))
    assert s[2].item() == 0.0 and int(q[2].abs().sum()) == 0  # zero row
    assert q[0, :6].tolist() == [127, 2, 0, 126, 4, -2]


def test_quant_strided_rows():
    announce("quant strided view")
    gen = torch.Generator().manual_seed(7)
    big = activations(12, 2048, gen).to(DEV)
    x = big[:, :1024]  # row stride 2048
    q, s = quant_per_token(x)
    q_ref, s_ref = orc.quant_per_token(f32(x))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


def test_quant_cfg2_full():
    """Config 2: [8192, 17408] bf16 with 0.1 % outliers, bit-exact."""
    announce("quant cfg2 8192x17408")
    gen = torch.Generator().manual_seed(0)
    _check_quant(activations(8192, 17408, gen))


def test_quant_rejects_bad_args():
    x = torch.zeros(4, 16, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(ValueError):
        quant_per_token(x.float())
    from minisgl_amd.kernel.lib import load

    rc = load().mw8_quant_per_token_bf16(None, 4, 16, 16, None, 16, None, None)
    assert rc == 1


@pytest.mark.parametrize("act", ["silu", "gelu"])
@pytest.mark.parametrize("R,two_d", [(1, 1536), (8, 1536), (300, 1536), (4, 34816), (3, 51200), (5, 32),
                                     (3, 2560), (2, 8208), (2, 12288), (37, 1536), (9, 1104)])
def test_act_and_mul_quant(act, R, two_d):
    announce(f"act {act} R={R} 2d={two_d}")
    gen = torch.Generator().manual_seed(R + two_d)
    x = activations(R, two_d, gen)
    q, s, a = act_and_mul_quant(x.to(DEV), act, return_act=True)
    torch.cuda.synchronize()
    a_ref = orc.silu_and_mul(f32(x)) if act == "silu" else orc.gelu_and_mul(f32(x))
    assert rel_l2(f32(a), a_ref) <= 1e-3
    # stage-wise: the requant of the GPU's own bf16 activation is bit-exact
    q_ref, s_ref = orc.quant_per_token(f32(a))
    np.testing.assert_array_equal(q.cpu().numpy(), q_ref)
    np.testing.assert_array_equal(s.cpu().numpy(), s_ref)


def test_act_rejects_odd_width():
    x = torch.zeros(2, 24, dtype=torch.bfloat16, device=DEV)
    with pytest.raises(MW8Error):
        act_and_mul_quant(x)
