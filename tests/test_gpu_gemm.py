"""GPU parity of the dense W8A8 GEMM (stream core for M <= 64, MFMA tile core
above) against the CPU oracle: int32 accumulators and bf16 outputs
bit-exact (the epilogue is the oracle's closed form, one rounding per op);
rel-L2 <= 1e-3 is checked as the contract bound as well."""

import numpy as np
import pytest
import torch

from helpers import announce, bf16_bits_equal, f32, rel_l2
from minisgl_amd.benchmark import linear_case
from minisgl_amd.kernel import MW8Error, gemm_w8a8, gemm_w8a8_i32, quant_per_token
from minisgl_amd.layers import (
    LinearColParallelMerged,
    LinearOProj,
    LinearQKVMerged,
    LinearReplicated,
    LinearRowParallel,
)
from oracle import w8a8 as orc

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _run_case(M, K, N, seed=0, bias=False, rows=None):
    c = linear_case(M, K, N, seed=seed, bias=bias)
    x = c["x"].to(DEV)
    w = c["w"].to(DEV)
    s_w = c["s_w"].to(DEV)
    b = c["bias"].to(DEV) if bias else None
    q, s_a = quant_per_token(x)
    acc = gemm_w8a8_i32(q, w)
    y = gemm_w8a8(q, s_a, w, s_w, b)
    torch.cuda.synchronize()
    # oracle on the same bytes (optionally on a row sample for large M)
    xs = f32(c["x"]) if rows is None else f32(c["x"][rows])
    q_ref, s_ref = orc.quant_per_token(xs)
    sel = slice(None) if rows is None else rows
    np.testing.assert_array_equal(q.cpu().numpy()[sel], q_ref)
    acc_ref = orc.gemm_i32(q_ref, c["w"].numpy())
    np.testing.assert_array_equal(acc.cpu().numpy()[sel], acc_ref)
    y_ref = orc.epilogue(acc_ref, s_ref, c["s_w"].numpy(), None if not bias else f32(c["bias"]))
    y_sel = y[sel] if rows is None else y[torch.as_tensor(rows, device=DEV)]
    assert rel_l2(f32(y_sel), y_ref) <= 1e-3
    eq = bf16_bits_equal(y_sel, y_ref)
    assert eq.all(), f"{(~eq).sum()} of {eq.size} bf16 outputs differ"


@pytest.mark.parametrize(
    "M,K,N",
    [
        (1, 128, 64), (3, 144, 100), (16, 1024, 6144), (17, 256, 192), (5, 2048, 80),
        (33, 1024, 128), (64, 1024, 320), (64, 4096, 512),
        (65, 512, 256), (100, 144, 100), (128, 1024, 1024), (200, 1040, 300), (512, 2048, 640),
    ],
)
def test_gemm_small_shapes(M, K, N):
    announce(f"gemm M={M} K={K} N={N}")
    _run_case(M, K, N, seed=M + K + N)


def test_gemm_cfg0():
    """Config 0: Qwen3-0.6B gate_up, M=16 K=1024 N=6144, seed 0."""
    announce("gemm cfg0")
    _run_case(16, 1024, 6144, seed=0)


@pytest.mark.parametrize("M", [1, 8, 64, 512])
@pytest.mark.parametrize("K,N", [(5120, 7168), (5120, 5120), (5120, 34816), (17408, 5120)])
def test_gemm_qwen3_14b(M, K, N):
    announce(f"gemm 14B M={M} K={K} N={N}")
    _run_case(M, K, N, seed=0)


@pytest.mark.parametrize("M", [4096, 8192])
@pytest.mark.parametrize("K,N", [(5120, 7168), (5120, 5120), (5120, 34816), (17408, 5120)])
def test_gemm_qwen3_14b_large_m_sampled(M, K, N):
    """Large M at all four Qwen3-14B shapes, under the tiling the library
    picks for each (gate_up M=8192 is the benchmark's dominant launch):
    every output is computed on the GPU; a sample of rows (first, last, and
    random rows, each row spanning every column tile) is checked."""
    announce(f"gemm 14B large M={M} K={K} N={N}")
    rng = np.random.default_rng(M + K + N)
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, 40, replace=False)]))
    _run_case(M, K, N, seed=0, rows=rows)


@pytest.mark.parametrize("M,N", [(192, 7168), (192, 5120), (384, 7168), (640, 7168), (768, 7168), (768, 5120)])
def test_gemm_mid_m_default_tiling_sampled(M, N):
    """qkv / o_proj between 192 and 768 rows under the automatic choice
    (64x64, 128x64 or 128x128 split-K tiles whose grid fits one wave, the
    256x128 ring where none does): a row sample checked bit-exact."""
    announce(f"gemm mid M={M} N={N}")
    rng = np.random.default_rng(M + N)
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, 30, replace=False)]))
    _run_case(M, 5120, N, seed=1, rows=rows)


def test_gemm_bias():
    announce("gemm bias")
    _run_case(16, 512, 384, seed=3, bias=True)
    _run_case(300, 512, 384, seed=4, bias=True)


def test_gemm_extremes():
    """All +127 x all -127 hits the closed form -K*127*127 in int32."""
    announce("gemm extremes")
    for M in (2, 130):
        K, N = 17408, 256
        a = torch.full((M, K), 127, dtype=torch.int8, device=DEV)
        w = torch.full((N, K), -127, dtype=torch.int8, device=DEV)
        acc = gemm_w8a8_i32(a, w)
        assert int(acc.min()) == int(acc.max()) == -K * 127 * 127


def test_gemm_workspace_reuse_and_zero_rows():
    """Two split-K calls in a row through one workspace (counters re-armed)."""
    announce("gemm workspace reuse")
    c1 = linear_case(8, 5120, 5120, seed=11)
    c2 = linear_case(3, 5120, 5120, seed=12)
    outs = []
    for c in (c1, c2, c1):
        q, s = quant_per_token(c["x"].to(DEV))
        outs.append(gemm_w8a8_i32(q, c["w"].to(DEV)).cpu())
    assert torch.equal(outs[0], outs[2])
    q_ref, _ = orc.quant_per_token(f32(c2["x"]))
    np.testing.assert_array_equal(outs[1].numpy(), orc.gemm_i32(q_ref, c2["w"].numpy()))
    empty = gemm_w8a8(torch.empty(0, 64, dtype=torch.int8, device=DEV), torch.empty(0, device=DEV),
                      torch.zeros(32, 64, dtype=torch.int8, device=DEV), torch.ones(32, device=DEV))
    assert empty.shape == (0, 32)


@pytest.mark.parametrize(
    "M,K,N", [(512, 5120, 7168), (300, 1280, 600), (1000, 2048, 1000), (4500, 768, 3840), (2304, 1280, 7168)]
)
def test_gemm_split_tail(M, K, N):
    """Tail-wave K split of the 256x256 tiling (forced): the last partial wave's tiles
    are cut into K ranges whose int32 partial tiles go to the workspace and
    are summed by the reduction kernel.  Bit-exact against the oracle (row
    sample for the larger cases) and against the launch without workspace,
    which runs the tiles whole."""
    import ctypes

    from minisgl_amd.kernel.lib import load

    announce(f"gemm split tail M={M} K={K} N={N}")
    lib = load()
    T = -(-M // 256) * -(-N // 256)
    r = T % 256
    sp = min(256 // r, K // 128, 16) if r else 0
    want_ws = r * sp * 65536 * 4 if sp >= 2 else 0
    lib.mw8_set_tuning(-1, 2, -1)  # the 8-wave 256x256 ring
    try:
        assert lib.mw8_gemm_workspace_bytes(M, N, K) == want_ws
        rows = None if M <= 1024 else np.unique(np.concatenate([[0, M - 1], np.arange(M - 300, M, 7)]))
        _run_case(M, K, N, seed=7, rows=rows)
        c = linear_case(M, K, N, seed=8)
        q, s = quant_per_token(c["x"].to(DEV))
        w = c["w"].to(DEV)
        split = gemm_w8a8_i32(q, w)
        whole = torch.empty_like(split)
        st = torch.cuda.current_stream().cuda_stream
        rc = lib.mw8_gemm_w8a8_i32(q.data_ptr(), w.data_ptr(), whole.data_ptr(), M, N, K, None, 0, st)
        assert rc == 0
        assert torch.equal(split, whole)
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


def test_gemm_rejects_bad_k():
    a = torch.zeros(4, 40, dtype=torch.int8, device=DEV)
    w = torch.zeros(8, 40, dtype=torch.int8, device=DEV)
    with pytest.raises(MW8Error):
        gemm_w8a8_i32(a, w)


def test_linear_layers_drop_in():
    """The Linear* drop-ins: constructor shapes as the reference, forward =
    quant + GEMM + epilogue, parity with the oracle."""
    announce("linear layers")
    gen = torch.Generator().manual_seed(5)
    layers = [
        LinearReplicated(256, 128, has_bias=False),
        LinearColParallelMerged(256, [192, 192], has_bias=False),
        LinearQKVMerged(256, head_dim=32, num_qo_heads=4, num_kv_heads=2, has_bias=True),
        LinearOProj(256, 256, has_bias=False),
        LinearRowParallel(256, 512, has_bias=False),
    ]
    for layer in layers:
        N, K = layer.weight.shape
        sd = {
            "weight": torch.randint(-127, 128, (N, K), generator=gen, dtype=torch.int8).to(DEV),
            "weight_scale": (torch.rand(N, generator=gen) * 1e-2).to(DEV),
        }
        if layer.bias is not None:
            sd["bias"] = torch.randn(N, generator=gen).to(torch.bfloat16).to(DEV)
        layer.load_state_dict(dict(sd))
        for M in (1, 70):
            x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
            y = layer.forward(x.to(DEV))
            y_ref, *_ = orc.linear_w8a8(
                f32(x), sd["weight"].cpu().numpy(), sd["weight_scale"].cpu().numpy(),
                None if layer.bias is None else f32(sd["bias"]),
            )
            assert bf16_bits_equal(y, y_ref).all()


@pytest.mark.parametrize("K", [8, 100, 1000, 4100])
def test_linear_layer_any_k(K):
    """K off the GEMM's 16-byte step, as F.linear takes it: the drop-in
    pads the weight (a cached copy) and the quantized rows with zeros, and
    the output equals the oracle's unpadded product bit for bit at decode
    and prefill batch sizes, with bias, after a weight reload (the cached
    copy is rebuilt), and through forward_quantized."""
    announce(f"linear any K={K}")
    gen = torch.Generator().manual_seed(K)
    N = 136
    layer = LinearReplicated(K, N, has_bias=True)
    for trial in range(2):  # the second load replaces the weight: the padded copy must follow
        sd = {
            "weight": torch.randint(-127, 128, (N, K), generator=gen, dtype=torch.int8).to(DEV),
            "weight_scale": (torch.rand(N, generator=gen) * 1e-2 + 1e-4).to(DEV),
            "bias": torch.randn(N, generator=gen).to(torch.bfloat16).to(DEV),
        }
        layer.load_state_dict(dict(sd))
        args = (sd["weight"].cpu().numpy(), sd["weight_scale"].cpu().numpy(), f32(sd["bias"]))
        for M in (1, 3, 64, 300):
            x = torch.randn(M, K, generator=gen).to(torch.bfloat16)
            y = layer.forward(x.to(DEV))
            y_ref, *_ = orc.linear_w8a8(f32(x), *args)
            eq = bf16_bits_equal(y, y_ref)
            assert eq.all(), f"trial {trial} M={M}: {(~eq).sum()} outputs differ"
        q, s = quant_per_token(x.to(DEV))
        y = layer.forward_quantized(q, s)
        assert bf16_bits_equal(y, y_ref).all(), "forward_quantized"


def _tuning_count(kind):
    from minisgl_amd.kernel.lib import load

    return int(load().mw8_tuning_count(kind))


@pytest.mark.parametrize(
    "M,K,N,bias",
    [(300, 640, 520, False), (257, 1024, 300, False), (129, 192, 64, False), (1000, 2048, 1000, False),
     (40, 1024, 520, False), (64, 2560, 1100, False), (130, 3072, 700, False),
     # K % 512 == 0: every in-block split-K configuration applies (partial row
     # tiles, N off the 16-column grid, column ranges narrower than the tile)
     (33, 1024, 1000, True), (64, 2048, 520, False), (100, 512, 36, True), (300, 1536, 1100, True),
     (1000, 1024, 2000, False), (2080, 512, 5120, True)],
)
def test_gemm_every_tile_config(M, K, N, bias):
    """Each tile configuration (forced through mw8_set_tuning) on ragged
    shapes; a configuration whose K granularity does not divide K falls
    back to the automatic choice.  33-64 rows take the tile core only when a
    tile configuration is forced; with few tiles the split-capable rings
    split every tile's K range."""
    from minisgl_amd.kernel.lib import load

    announce(f"gemm all tile cfgs M={M} K={K} N={N} bias={bias}")
    c = linear_case(M, K, N, seed=M, bias=bias)
    q, s = quant_per_token(c["x"].to(DEV))
    w, s_w = c["w"].to(DEV), c["s_w"].to(DEV)
    b = c["bias"].to(DEV) if bias else None
    q_ref, s_ref = orc.quant_per_token(f32(c["x"]))
    acc_ref = orc.gemm_i32(q_ref, c["w"].numpy())
    y_ref = orc.epilogue(acc_ref, s_ref, c["s_w"].numpy(), f32(c["bias"]) if bias else None)
    lib = load()
    try:
        for cfg in range(_tuning_count(1)):
            lib.mw8_set_tuning(-1, cfg, -1)
            np.testing.assert_array_equal(gemm_w8a8_i32(q, w).cpu().numpy(), acc_ref, err_msg=f"cfg {cfg}")
            assert bf16_bits_equal(gemm_w8a8(q, s, w, s_w, b), y_ref).all(), f"cfg {cfg}"
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


@pytest.mark.parametrize("K", [128, 256, 384, 640])
@pytest.mark.parametrize("M,N", [(1040, 1040), (4096, 2048)])
def test_gemm_rings_short_k(M, K, N):
    """Every tile configuration at 1-5 K stages of 128 bytes: the prologue
    and tail of the rings whose weight stages run ahead of their A stages
    (fewer stages than ring slots, whole tiles at 4096 x 2048 and K-split
    tiles at 1040 x 1040), against the oracle."""
    from minisgl_amd.kernel.lib import load

    announce(f"gemm rings short K M={M} K={K} N={N}")
    c = linear_case(M, K, N, seed=K + N, bias=True)
    q, s = quant_per_token(c["x"].to(DEV))
    w, s_w, b = c["w"].to(DEV), c["s_w"].to(DEV), c["bias"].to(DEV)
    q_ref, s_ref = orc.quant_per_token(f32(c["x"]))
    acc_ref = orc.gemm_i32(q_ref, c["w"].numpy())
    y_ref = orc.epilogue(acc_ref, s_ref, c["s_w"].numpy(), f32(c["bias"]))
    lib = load()
    try:
        for cfg in range(_tuning_count(1)):
            lib.mw8_set_tuning(-1, cfg, -1)
            np.testing.assert_array_equal(gemm_w8a8_i32(q, w).cpu().numpy(), acc_ref, err_msg=f"cfg {cfg}")
            assert bf16_bits_equal(gemm_w8a8(q, s, w, s_w, b), y_ref).all(), f"cfg {cfg}"
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


@pytest.mark.parametrize(
    "M,K,N",
    [(1, 1344, 336), (5, 1344, 336), (16, 1344, 336), (17, 1344, 336), (33, 1344, 336), (64, 1344, 336),
     (1, 1328, 200), (8, 1328, 200), (40, 1328, 200),  # K % 64 == 48: partial last step
     (3, 4160, 72), (16, 4160, 72),  # 65 steps: several pipelined batches per wave
     # CU-balanced grids: uneven row ranges of 1-32 rows per block
     (1, 1344, 5000), (16, 1344, 8200), (32, 2048, 4100), (7, 1024, 16400),
     # shared-token core (K % 256 == 0, up to 64 tokens): 9 waves with a ragged
     # last wave, one wave of 2-3 rows, 10 waves (3 stages), a grid of 512 blocks
     (8, 2048, 34820), (16, 512, 600), (2, 256, 40000), (4, 768, 49200),
     # and 2-4 token groups: 17-64 tokens, ragged M
     (20, 1024, 20000), (48, 512, 36000), (64, 256, 9000)],
)
def test_gemm_every_decode_config(M, K, N):
    from minisgl_amd.kernel.lib import load

    announce(f"gemm all decode cfgs M={M} K={K} N={N}")
    c = linear_case(M, K, N, seed=M)
    q, s = quant_per_token(c["x"].to(DEV))
    w, s_w = c["w"].to(DEV), c["s_w"].to(DEV)
    q_ref, s_ref = orc.quant_per_token(f32(c["x"]))
    acc_ref = orc.gemm_i32(q_ref, c["w"].numpy())
    y_ref = orc.epilogue(acc_ref, s_ref, c["s_w"].numpy())
    lib = load()
    try:
        for cfg in range(_tuning_count(0)):
            lib.mw8_set_tuning(cfg, -1, -1)
            np.testing.assert_array_equal(gemm_w8a8_i32(q, w).cpu().numpy(), acc_ref, err_msg=f"cfg {cfg}")
            assert bf16_bits_equal(gemm_w8a8(q, s, w, s_w), y_ref).all(), f"cfg {cfg}"
    finally:
        lib.mw8_set_tuning(-1, -1, -1)


@pytest.mark.parametrize(
    "M,K,N,bias",
    [(4100, 768, 4104, True), (2080, 1024, 8200, False), (4096, 5120, 7168, False), (8192, 896, 2056, True)],
)
def test_gemm_stream_walk(M, K, N, bias):
    """The pipelined persistent walk (tile configuration 7, forced) on shapes
    it takes (at least one 256 x 256 tile per CU, K >= 768), ragged in M and
    N, with and without bias: bit-identical to the one-tile 256 x 256 ring
    (configuration 2) on every output, and bit-exact against the oracle on a
    row sample (first and last rows, rows of the last partial tile)."""
    from minisgl_amd.kernel.lib import load

    announce(f"gemm stream walk M={M} K={K} N={N} bias={bias}")
    c = linear_case(M, K, N, seed=M + N, bias=bias)
    q, s = quant_per_token(c["x"].to(DEV))
    w, s_w = c["w"].to(DEV), c["s_w"].to(DEV)
    b = c["bias"].to(DEV) if bias else None
    lib = load()
    try:
        lib.mw8_set_tuning(-1, 7, -1)
        assert lib.mw8_gemm_kernel_name(M, N, K).decode().startswith("stream_gemm_kernel")
        y_stream = gemm_w8a8(q, s, w, s_w, b)
        lib.mw8_set_tuning(-1, 2, -1)
        y_tile = gemm_w8a8(q, s, w, s_w, b)
    finally:
        lib.mw8_set_tuning(-1, -1, -1)
    torch.cuda.synchronize()
    assert torch.equal(y_stream.view(torch.int16), y_tile.view(torch.int16))
    rows = np.unique(np.r_[0, 1, M - 1, np.arange(M - 40, M, 3), np.linspace(0, M - 1, 24).astype(int)])
    q_ref, s_ref = orc.quant_per_token(f32(c["x"][rows]))
    y_ref = orc.epilogue(orc.gemm_i32(q_ref, c["w"].numpy()), s_ref, c["s_w"].numpy(),
                         f32(c["bias"]) if bias else None)
    assert bf16_bits_equal(y_stream[torch.as_tensor(rows, device=DEV)], y_ref).all()


@pytest.mark.parametrize("K,N", [(5120, 5120), (5120, 7168), (1024, 6144), (1040, 520), (2048, 2056), (8192, 1024), (12288, 520)])
def test_linear_bf16_fused_quant(K, N):
    """The one-launch decode linear (mw8_linear_bf16_w8a8: per-token
    quantization inside the decode GEMM) equals quant_per_token followed by
    gemm_w8a8 bit for bit, for 1-16 tokens, under every decode configuration
    that takes the shape; rows with a stride past K, an all-zero row, a row
    of tiny values (absmax below 2^-60: the division path of the quantizer,
    beside rows on the reciprocal path in the same wave), x20 outliers and a
    bias; and the oracle on every row."""
    from minisgl_amd.kernel import linear_bf16_supported, linear_bf16_w8a8
    from minisgl_amd.kernel.lib import load

    announce(f"linear bf16 fused quant K={K} N={N}")
    lib = load()
    gen = torch.Generator().manual_seed(K + N)
    w = torch.randint(-127, 128, (N, K), generator=gen, dtype=torch.int8)
    s_w = torch.rand(N, generator=gen) * 9e-3 + 1e-3
    bias = torch.randn(N, generator=gen).to(torch.bfloat16)
    wd, swd, bd = w.to(DEV), s_w.to(DEV), bias.to(DEV)
    for M in (1, 2, 3, 4, 8, 16):
        buf = torch.randn(M, K + 64, generator=gen) * 2
        buf[:, :K][torch.rand(M, K, generator=gen) < 1e-3] *= 20
        if M >= 3:
            buf[1] = 0.0  # all-zero row: s = 0, q = 0
        if M >= 4:
            buf[2] *= 2.0**-70  # absmax below 2^-60: the division path
        xb = buf.to(torch.bfloat16)
        x = xb.to(DEV)[:, :K]  # row stride K + 64
        for b, bref in ((None, None), (bd, f32(bias))):
            q, s = quant_per_token(x.contiguous())
            want = gemm_w8a8(q, s, wd, swd, b)
            q_ref, s_ref = orc.quant_per_token(f32(xb[:, :K]))
            y_ref = orc.epilogue(orc.gemm_i32(q_ref, w.numpy()), s_ref, s_w.numpy(), bref)
            assert bf16_bits_equal(want, y_ref).all(), f"reference path M={M}"
            ran = 0
            try:
                for cfg in [-1] + list(range(_tuning_count(0))):
                    lib.mw8_set_tuning(cfg, -1, -1)
                    if not linear_bf16_supported(M, N, K):
                        continue
                    got = linear_bf16_w8a8(x, wd, swd, b)
                    assert torch.equal(got.view(torch.int16), want.view(torch.int16)), f"M={M} cfg={cfg}"
                    ran += 1
            finally:
                lib.mw8_set_tuning(-1, -1, -1)
            if M <= 4 and M * K <= 4 * 5120:
                assert ran >= 2, f"M={M}: the default and at least one forced configuration take the shape"
            elif M * K <= 4 * 5120:
                assert ran >= 1, f"M={M}: a configuration takes the shape"
            else:
                assert ran == 0, f"M={M}: past the fused form's element budget"


@pytest.mark.parametrize("M", [1, 4])
def test_linear_layer_decode_takes_the_fused_path(M):
    """LinearOProj.forward on a decode batch of bf16 rows runs the one-launch
    fused linear (no separate quantizer call) and matches the oracle."""
    import minisgl_amd.layers.linear as lin

    announce(f"linear layer fused decode path M={M}")
    gen = torch.Generator().manual_seed(9)
    layer = LinearOProj(5120, 5120, has_bias=False)
    sd = {"weight": torch.randint(-127, 128, (5120, 5120), generator=gen, dtype=torch.int8),
          "weight_scale": torch.rand(5120, generator=gen) * 1e-2}
    layer.load_state_dict({k: v.to(DEV) for k, v in sd.items()})
    x = torch.randn(M, 5120, generator=gen).to(torch.bfloat16)

    def _no_quant(*a, **kw):
        raise AssertionError("the decode forward called the separate quantizer")

    orig = lin.quant_per_token
    lin.quant_per_token = _no_quant
    try:
        y = layer.forward(x.to(DEV))
    finally:
        lin.quant_per_token = orig
    y_ref, *_ = orc.linear_w8a8(f32(x), sd["weight"].numpy(), sd["weight_scale"].numpy())
    assert bf16_bits_equal(y, y_ref).all()


def test_gemm_concurrent_streams():
    """Two K-split GEMMs (down at 512 rows: 40 tiles in 6 K ranges, 60 MiB of
    int32 partial tiles each) in flight at once on two streams, then the same
    pair on one stream: bit-identical.  Each call's partial tiles have a
    buffer of their own (torch's caching allocator keys blocks by stream)."""
    from minisgl_amd.kernel.lib import load

    announce("gemm concurrent streams")
    M, K, N = 512, 17408, 5120
    assert load().mw8_gemm_workspace_bytes(M, N, K) > 0, "the case must take the K split"
    cases = [linear_case(M, K, N, seed=s) for s in (21, 22)]
    ins = []
    for c in cases:
        q, s = quant_per_token(c["x"].to(DEV))
        ins.append((q, s, c["w"].to(DEV), c["s_w"].to(DEV)))
    torch.cuda.synchronize()
    want = [gemm_w8a8(*a) for a in ins]
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    got = [None, None]
    for _ in range(3):
        for i, st in enumerate(streams):
            st.wait_stream(torch.cuda.current_stream())
            with torch.cuda.stream(st):
                got[i] = gemm_w8a8(*ins[i])
        for st in streams:
            torch.cuda.current_stream().wait_stream(st)
        torch.cuda.synchronize()
        for i in range(2):
            assert torch.equal(got[i].view(torch.int16), want[i].view(torch.int16)), f"stream {i}"
