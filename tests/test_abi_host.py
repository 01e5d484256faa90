"""CPU tests of the drop-in boundary: libmw8.so loads and exports every
symbol include/mw8.h declares, argument validation returns the documented
error codes before any GPU work, and the host-side mirror of the reference
interface (registry, BaseOP state dicts, layer shapes, MoE regimes)
behaves like the reference.  No GPU compute happens here."""

import ctypes
import os
import re

import pytest
import torch

from minisgl_amd.kernel import lib as mw8lib

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "mw8.h")
CALIB_HEADER = os.path.join(ROOT, "include", "mw8_calib.h")


def _declared(path=HEADER):
    text = open(path).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(mw8_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def lib():
    return mw8lib.load()


def test_header_declares_entry_points():
    names = _declared()
    for n in ("mw8_quant_per_token_bf16", "mw8_gemm_w8a8_bf16", "mw8_moe_align_block_size",
              "mw8_moe_gemm_w8a8_bf16", "mw8_moe_sum_reduce_bf16", "mw8_topk_softmax"):
        assert n in names


def test_library_exports_every_declared_symbol(lib):
    raw = ctypes.CDLL(mw8lib.LIB_PATH)
    missing = [n for n in _declared() if not hasattr(raw, n)]
    assert not missing, missing


def test_binding_covers_header():
    assert set(_declared()) == set(mw8lib.SIGNATURES)


def test_measurement_kernels_are_a_library_of_their_own():
    """The benchmark's measurement kernels (include/mw8_calib.h) are exported
    by libmw8_calib.so and bound by kernel/lib.py, and the product library
    exports none of them."""
    names = _declared(CALIB_HEADER)
    assert set(names) == set(mw8lib.CALIB_SIGNATURES)
    calib = ctypes.CDLL(mw8lib.CALIB_PATH)
    assert [n for n in names if not hasattr(calib, n)] == []
    product = ctypes.CDLL(mw8lib.LIB_PATH)
    assert [n for n in names if hasattr(product, n)] == []
    clib = mw8lib.load_calib()
    assert clib.mw8_calib_sink_len() == 2048 * 256  # the read grid, the larger of the kernels
    assert clib.mw8_calib_read(None, 1 << 20, None, 0, None) == 1  # MW8_ERR_ARG before any launch
    assert b"null pointer" in clib.mw8_calib_last_error()


def test_version_and_pure_host_helpers(lib):
    assert lib.mw8_version() >= 100
    # python/minisgl/moe/fused.py:73: numel + (E + 1) * (B - 1)
    assert lib.mw8_moe_align_max_padded(12, 5, 4) == 27
    assert lib.mw8_moe_align_max_padded(128, 129, 16) == 128 + 129 * 15
    assert lib.mw8_gemm_workspace_bytes(1, 5120, 5120) == 0
    # tail split of 256x256 tilings (forced): r = T mod 256 tail tiles, sp = min(256 // r,
    # K / 128, 16) K ranges each, one int32 256x256 partial tile per (tile, range)
    lib.mw8_set_tuning(-1, 2, -1)
    try:
        assert lib.mw8_gemm_workspace_bytes(1024, 34816, 5120) == 32 * 8 * 256 * 256 * 4
        assert lib.mw8_gemm_workspace_bytes(4096, 5120, 5120) == 64 * 4 * 256 * 256 * 4
    finally:
        lib.mw8_set_tuning(-1, -1, -1)
    # automatic: N = 5120 at 4096 rows runs 256x320 tiles, 256 of them (no split)
    assert lib.mw8_gemm_kernel_name(4096, 5120, 5120) == b"tile3_gemm_kernel<256, 320, 128, 2, 4, 2>"
    assert lib.mw8_gemm_workspace_bytes(4096, 5120, 5120) == 0
    assert lib.mw8_gemm_kernel_name(8192, 34816, 5120) == b"tile3_gemm_kernel<256, 256, 128, 2, 4, 2>"
    assert lib.mw8_gemm_workspace_bytes(8192, 34816, 5120) == 0  # 4352 tiles: whole waves
    assert lib.mw8_gemm_workspace_bytes(4096, 7168, 5120) == 0   # 192 tail tiles: no split
    assert lib.mw8_gemm_workspace_bytes(512, 5120, 5120 + 64) == 0  # K % 128 != 0
    assert lib.mw8_gemm_workspace_bytes(512, 7168, 5120) == 0  # 128x128 ring (no split) chosen
    # the 64x128 ring (forced): 272 tiles, 16 in the tail, 16 K ranges each
    lib.mw8_set_tuning(-1, 5, -1)
    try:
        assert lib.mw8_gemm_workspace_bytes(64, 34816, 5120) == 16 * 16 * 64 * 128 * 4
        assert lib.mw8_gemm_workspace_bytes(40, 1024, 1024) == 8 * 8 * 64 * 128 * 4  # all 8 tiles split
    finally:
        lib.mw8_set_tuning(-1, -1, -1)
    assert lib.mw8_gemm_workspace_bytes(32, 34816, 5120) == 0  # decode core


def test_tuning_override_is_per_thread(lib):
    """A tuning override changes the choice of the thread that set it only:
    another thread, before and while it holds, sees the automatic tiling."""
    import threading

    auto = b"tile3_gemm_kernel<256, 256, 128, 2, 4, 2>"
    seen = []
    lib.mw8_set_tuning(-1, 5, -1)
    try:
        assert lib.mw8_gemm_kernel_name(8192, 34816, 5120) != auto
        t = threading.Thread(target=lambda: seen.append(lib.mw8_gemm_kernel_name(8192, 34816, 5120)))
        t.start()
        t.join()
    finally:
        lib.mw8_set_tuning(-1, -1, -1)
    assert seen == [auto]
    assert lib.mw8_gemm_kernel_name(8192, 34816, 5120) == auto


def test_moe_gemm_sum_supported_sizes(lib):
    """The fused down-projection + slot sum keeps its routing tables in LDS:
    every decode batch of config 3 (up to E = 128 tokens x top-8, sorted
    positions numel + (E + 1) * 15) fits, and so does E = 256 at 1024 pairs;
    more pairs, more sorted positions than one prologue pass loads, more than
    256 experts or negative sizes do not."""
    sup = lib.mw8_moe_gemm_sum_supported
    for m in (1, 16, 64, 128):
        P = m * 8
        assert sup(lib.mw8_moe_align_max_padded(P, 128, 16), P, 128) == 1
    assert sup(lib.mw8_moe_align_max_padded(1024, 256, 16), 1024, 256) == 1
    assert sup(lib.mw8_moe_align_max_padded(2048, 256, 16), 2048, 256) == 0
    assert sup(6160, 64, 8) == 0
    assert sup(lib.mw8_moe_align_max_padded(4096, 128, 16), 4096, 128) == 0
    assert sup(1024, 64, 257) == 0
    assert sup(-16, 8, 8) == 0 and sup(16, -8, 8) == 0


def test_workspace_bound_and_tuning_counts(lib):
    """mw8_gemm_workspace_max_bytes bounds every plan (r * sp <= S slots of
    the largest split tile), so one reservation never has to grow; the
    tuning tables have the documented sizes.  Without a GPU the library
    plans for 256 CUs."""
    mx = lib.mw8_gemm_workspace_max_bytes()
    assert mx == 256 * 256 * 256 * 4
    # the allocation-free entry's static scratch (64 MiB) holds every plan on 256 CUs
    assert mx <= 64 << 20
    counts = [lib.mw8_tuning_count(k) for k in range(4)]
    assert counts == [10, 13, 3, 3] and lib.mw8_tuning_count(9) == 0
    worst = 0
    try:
        for tile in range(-1, counts[1]):
            lib.mw8_set_tuning(-1, tile, -1)
            for M in (33, 40, 64, 65, 100, 128, 200, 256, 300, 512, 1000, 2080, 4096, 8192):
                for N, K in ((5120, 5120), (7168, 5120), (34816, 5120), (5120, 17408), (1000, 1024), (64, 128)):
                    worst = max(worst, lib.mw8_gemm_workspace_bytes(M, N, K))
    finally:
        lib.mw8_set_tuning(-1, -1, -1)
    assert 0 < worst <= mx


def test_linear_bf16_supported_shapes(lib):
    """The one-launch decode linear takes up to 16 tokens and 4 x 5120
    elements of x, where the decode core's waves stream at most 6 K stages
    of 256 bytes and one ring slot holds a wave's range of the int8 rows
    (planned for 256 CUs without a GPU): o_proj / qkv of Qwen3-14B at 1-4
    tokens, not at 5 tokens; config 0 (16 tokens, K = 1024), not 17 tokens;
    not the K = 17408 down projection, not K % 16 != 0."""
    sup = lib.mw8_linear_bf16_supported
    for M in (1, 2, 3, 4):
        assert sup(M, 5120, 5120) == 1 and sup(M, 7168, 5120) == 1
    assert sup(5, 5120, 5120) == 0 and sup(0, 5120, 5120) == 0
    assert sup(16, 6144, 1024) == 1 and sup(17, 6144, 1024) == 0
    assert sup(1, 5120, 17408) == 0
    assert sup(1, 5120, 5128) == 0


FAKE_A, FAKE_B, FAKE_C = 4096, 8192, 12288  # aligned non-null stand-ins: never dereferenced


def test_argument_errors_return_codes(lib):
    E = {v: k for k, v in mw8lib.ERROR_NAMES.items()}
    assert lib.mw8_quant_per_token_bf16(None, 4, 16, 16, None, 16, None, None) == E["MW8_ERR_ARG"]
    assert b"null" in lib.mw8_last_error()
    assert lib.mw8_quant_per_token_bf16(FAKE_A, 4, 16, 8, FAKE_B, 16, FAKE_C, None) == E["MW8_ERR_SHAPE"]
    # the one-launch decode linear: null operand, too many tokens, unaligned row stride
    lin = lib.mw8_linear_bf16_w8a8
    assert lin(None, 5120, FAKE_B, FAKE_C, None, FAKE_A, 1, 5120, 5120, None) == E["MW8_ERR_ARG"]
    assert lin(FAKE_A, 5120, FAKE_B, FAKE_C, None, FAKE_A, 5, 5120, 5120, None) == E["MW8_ERR_SHAPE"]
    assert lin(FAKE_A, 5124, FAKE_B, FAKE_C, None, FAKE_A, 2, 5120, 5120, None) == E["MW8_ERR_ALIGN"]
    # the gate_up GEMM with the activation: null operand, bad activation, a decode shape, I % 8 != 0
    act = lib.mw8_gemm_act_w8a8_bf16
    assert act(None, FAKE_B, FAKE_C, FAKE_B, 0, FAKE_A, 2080, 25600, 5120, None, 0, None) == E["MW8_ERR_ARG"]
    assert act(FAKE_A, FAKE_B, FAKE_C, FAKE_B, 2, FAKE_A, 2080, 25600, 5120, None, 0, None) == E["MW8_ERR_ARG"]
    assert act(FAKE_A, FAKE_B, FAKE_C, FAKE_B, 0, FAKE_A, 1, 25600, 5120, None, 0, None) == E["MW8_ERR_SHAPE"]
    assert act(FAKE_A, FAKE_B, FAKE_C, FAKE_B, 0, FAKE_A, 2080, 25604, 5120, None, 0, None) == E["MW8_ERR_SHAPE"]
    assert lib.mw8_gemm_act_supported(2080, 25600, 5120) == 1 and lib.mw8_gemm_act_supported(8, 25600, 5120) == 0
    assert lib.mw8_gemm_act_workspace_bytes(2080, 25600, 5120) > 0  # the short last wave splits along K
    # K % 16 != 0
    rc = lib.mw8_gemm_w8a8_i32(FAKE_A, FAKE_B, FAKE_C, 4, 8, 40, None, 0, None)
    assert rc == E["MW8_ERR_SHAPE"] and b"multiple of 16" in lib.mw8_last_error()
    # misaligned operand
    rc = lib.mw8_gemm_w8a8_i32(FAKE_A + 4, FAKE_B, FAKE_C, 4, 8, 64, None, 0, None)
    assert rc == E["MW8_ERR_ALIGN"]
    # K beyond the exact int32 accumulation bound
    rc = lib.mw8_gemm_w8a8_i32(FAKE_A, FAKE_B, FAKE_C, 4, 8, 1 << 18, None, 0, None)
    assert rc == E["MW8_ERR_SHAPE"]
    # bf16 epilogue without scales
    rc = lib.mw8_gemm_w8a8_bf16(FAKE_A, None, FAKE_B, None, None, FAKE_C, 4, 8, 64, None, 0, None)
    assert rc == E["MW8_ERR_ARG"]
    assert lib.mw8_act_and_mul_quant_bf16(FAKE_A, 4, 24, 0, FAKE_B, FAKE_C, None, None) == E["MW8_ERR_SHAPE"]
    assert lib.mw8_act_and_mul_quant_bf16(FAKE_A, 4, 32, 7, FAKE_B, FAKE_C, None, None) == E["MW8_ERR_ARG"]
    assert lib.mw8_topk_softmax(FAKE_A, 1, 4, 8, 9, 1, FAKE_B, FAKE_C, None) == E["MW8_ERR_SHAPE"]
    assert lib.mw8_moe_align_block_size(FAKE_A, 16, 600, 16, FAKE_B, FAKE_C, FAKE_A, None) == E["MW8_ERR_SHAPE"]
    rc = lib.mw8_moe_gemm_w8a8_i32(FAKE_A, FAKE_B, FAKE_C, FAKE_C, FAKE_C, 64, 1, 16, 64, 64, 4, 48,
                                   FAKE_A, None)
    assert rc == E["MW8_ERR_SHAPE"]  # block size 48 unsupported
    # small-batch preparation: M * topk > 1024, H % 8 != 0, slots < E, a null output
    prep = lib.mw8_moe_prepare_small
    assert prep(FAKE_A, 1, 129, 16, 8, 1, FAKE_B, 64, FAKE_C, FAKE_C, FAKE_C, FAKE_C, 17, 16,
                FAKE_A, FAKE_B, FAKE_C, None) == E["MW8_ERR_SHAPE"]
    assert prep(FAKE_A, 1, 4, 16, 8, 1, FAKE_B, 60, FAKE_C, FAKE_C, FAKE_C, FAKE_C, 17, 16,
                FAKE_A, FAKE_B, FAKE_C, None) == E["MW8_ERR_SHAPE"]
    assert prep(FAKE_A, 1, 4, 16, 8, 1, FAKE_B, 64, FAKE_C, FAKE_C, FAKE_C, FAKE_C, 15, 16,
                FAKE_A, FAKE_B, FAKE_C, None) == E["MW8_ERR_SHAPE"]
    assert prep(FAKE_A, 1, 4, 16, 8, 1, FAKE_B, 64, None, FAKE_C, FAKE_C, FAKE_C, 17, 16,
                FAKE_A, FAKE_B, FAKE_C, None) == E["MW8_ERR_ARG"]
    assert lib.mw8_moe_sum_reduce_bf16(FAKE_A, 4, 8, 12, FAKE_B, None) == E["MW8_ERR_SHAPE"]
    # strided RMSNorm: H % 8 != 0, stride below inner * H, null weight
    assert lib.mw8_rmsnorm_strided_bf16(FAKE_A, 96, FAKE_A, 96, FAKE_B, 1e-6, 4, 8, 12, None) == E["MW8_ERR_SHAPE"]
    assert lib.mw8_rmsnorm_strided_bf16(FAKE_A, 64, FAKE_A, 64, FAKE_B, 1e-6, 4, 8, 16, None) == E["MW8_ERR_SHAPE"]
    assert lib.mw8_rmsnorm_strided_bf16(FAKE_A, 256, FAKE_A, 256, None, 1e-6, 4, 8, 16, None) == E["MW8_ERR_ARG"]
    assert lib.mw8_rmsnorm_strided_bf16(FAKE_A + 2, 256, FAKE_A, 256, FAKE_B, 1e-6, 4, 8, 16, None) == E["MW8_ERR_ALIGN"]
    # down-projection with the slot sum: null operand, pairs not a multiple of top_k, LDS tables too large
    gs = lib.mw8_moe_gemm_sum_w8a8_bf16
    assert gs(None, FAKE_B, FAKE_A, FAKE_B, FAKE_C, FAKE_C, FAKE_C, 2944, None, 8, 1024, 2048, 768, 128,
              FAKE_A, None) == E["MW8_ERR_ARG"]
    assert gs(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, FAKE_C, FAKE_C, 2944, None, 8, 1020, 2048, 768, 128,
              FAKE_A, None) == E["MW8_ERR_SHAPE"]
    assert gs(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, FAKE_C, FAKE_C, 8000, None, 8, 4000, 2048, 768, 128,
              FAKE_A, None) == E["MW8_ERR_SHAPE"] and b"LDS" in lib.mw8_last_error()
    assert gs(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, FAKE_C, FAKE_C, 2944, None, 8, 1024, 2048, 760, 128,
              FAKE_A, None) == E["MW8_ERR_SHAPE"]  # K % 16 != 0
    # router-id grouped GEMMs: more than 48 tokens, null ids, pairs not a multiple of top_k,
    # one scale without the other, K % 16 != 0, more expert units than the slot-sum tables hold
    for fn in (lib.mw8_moe_gemm_topk_w8a8_bf16, lib.mw8_moe_gemm_sum_topk_w8a8_bf16):
        assert fn(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, None, 8, 49 * 8, 2048, 768, 128, FAKE_A,
                  None) == E["MW8_ERR_SHAPE"] and b"48 tokens" in lib.mw8_last_error()
        assert fn(FAKE_A, FAKE_B, FAKE_A, FAKE_B, None, None, 8, 128, 2048, 768, 128, FAKE_A,
                  None) == E["MW8_ERR_ARG"]
        assert fn(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, None, 8, 100, 2048, 768, 128, FAKE_A,
                  None) == E["MW8_ERR_SHAPE"]
        assert fn(FAKE_A, FAKE_B, FAKE_A, None, FAKE_C, None, 8, 128, 2048, 768, 128, FAKE_A,
                  None) == E["MW8_ERR_ARG"]
        assert fn(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, None, 8, 128, 2048, 760, 128, FAKE_A,
                  None) == E["MW8_ERR_SHAPE"]
        assert fn(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, None, 8, 0, 2048, 768, 128, FAKE_A, None) == 0
    assert lib.mw8_moe_gemm_sum_topk_w8a8_bf16(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, None, 8, 128, 2048,
                                              768, 400, FAKE_A, None) == E["MW8_ERR_SHAPE"]
    assert lib.mw8_moe_gemm_sum_topk_w8a8_bf16(FAKE_A, FAKE_B, FAKE_A, FAKE_B, FAKE_C, None, 8, 48 * 8, 2048,
                                              768, 129, FAKE_A, None) == E["MW8_ERR_SHAPE"]  # 3 x 129 > 384 units
    # empty problems are no-ops
    assert lib.mw8_gemm_w8a8_i32(FAKE_A, FAKE_B, FAKE_C, 0, 8, 64, None, 0, None) == 0


def test_ops_refuse_cpu_tensors():
    """No CPU fallback: the product path raises on host tensors."""
    from minisgl_amd.kernel import gemm_w8a8, quant_per_token

    with pytest.raises(ValueError, match="GPU"):
        quant_per_token(torch.zeros(2, 16, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="GPU"):
        gemm_w8a8(torch.zeros(2, 16, dtype=torch.int8), torch.ones(2), torch.zeros(4, 16, dtype=torch.int8), torch.ones(4))


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(RuntimeError, match="not found"):
        mw8lib.load.__wrapped__(str(tmp_path / "libmw8.so"))


# ------------------------------------------------------------ host interface
def test_registry_semantics():
    from minisgl_amd.moe import SUPPORTED_MOE_BACKENDS, create_moe_backend
    from minisgl_amd.moe.fused import FusedMoeW8A8
    from minisgl_amd.utils import Registry

    assert "fused_w8a8" in SUPPORTED_MOE_BACKENDS.supported_names()
    assert isinstance(create_moe_backend("fused_w8a8"), FusedMoeW8A8)
    with pytest.raises(KeyError):
        SUPPORTED_MOE_BACKENDS["nope"]
    r = Registry("X")
    r.register("a")(1)
    with pytest.raises(KeyError):
        r.register("a")
    import argparse

    with pytest.raises(argparse.ArgumentTypeError):
        r.assert_supported(["a", "b"])


def test_linear_shapes_match_reference_constructors():
    from minisgl_amd.layers import (
        LinearColParallelMerged,
        LinearOProj,
        LinearQKVMerged,
        LinearReplicated,
        LinearRowParallel,
    )

    # Qwen3-14B: hidden 5120, 40 q heads / 8 kv heads, head_dim 128, intermediate 17408
    qkv = LinearQKVMerged(5120, 128, 40, 8, has_bias=False)
    assert qkv.weight.shape == (7168, 5120) and qkv.weight.dtype == torch.int8
    assert qkv.weight_scale.shape == (7168,) and qkv.weight_scale.dtype == torch.float32
    assert qkv.bias is None
    gu = LinearColParallelMerged(5120, [17408, 17408], has_bias=False)
    assert gu.weight.shape == (34816, 5120)
    assert LinearRowParallel(17408, 5120, False).weight.shape == (5120, 17408)
    assert LinearOProj(5120, 5120, False).weight.shape == (5120, 5120)
    b = LinearReplicated(16, 8, has_bias=True)
    assert b.bias.dtype == torch.bfloat16 and b.bias.shape == (8,)


def test_state_dict_roundtrip_and_checks():
    from minisgl_amd.layers import LinearQKVMerged, MoELayer

    layer = LinearQKVMerged(64, 16, 2, 1, has_bias=True)
    sd = layer.state_dict(prefix="model.layers.0.qkv_proj")
    assert set(sd) == {"model.layers.0.qkv_proj.weight", "model.layers.0.qkv_proj.weight_scale",
                       "model.layers.0.qkv_proj.bias"}
    new = {k: torch.zeros_like(v) for k, v in sd.items()}
    layer.load_state_dict({k.split("qkv_proj.")[1]: v for k, v in new.items()})
    with pytest.raises(AssertionError):  # dtype mismatch (bf16 weight into an int8 slot)
        layer.load_state_dict({"weight": torch.zeros(64, 64, dtype=torch.bfloat16),
                               "weight_scale": torch.zeros(64), "bias": torch.zeros(64, dtype=torch.bfloat16)})
    with pytest.raises(RuntimeError, match="Unexpected"):
        layer.load_state_dict({"weight": torch.zeros(64, 64, dtype=torch.int8), "weight_scale": torch.zeros(64),
                               "bias": torch.zeros(64, dtype=torch.bfloat16), "extra": torch.zeros(1)})
    moe = MoELayer(8, 2, 64, 32)
    assert {k: tuple(v.shape) for k, v in moe.state_dict().items()} == {
        "gate_up_proj": (8, 64, 64), "down_proj": (8, 64, 32),
        "gate_up_scale": (8, 64), "down_scale": (8, 64),
    }


def test_moe_default_config_regimes():
    from minisgl_amd.moe.fused import get_default_config, try_get_optimal_moe_config

    # python/minisgl/moe/fused.py:92-113: M <= E -> small blocks
    assert get_default_config(16, 128, 2048, 2048, 8)["BLOCK_SIZE_M"] == 16
    assert get_default_config(256, 128, 2048, 2048, 8)["BLOCK_SIZE_M"] == 64
    assert try_get_optimal_moe_config((128, 1536, 2048), (128, 2048, 768), 8, 4096)["BLOCK_SIZE_M"] == 64


def test_moe_layer_needs_context():
    from minisgl_amd.core import reset_global_ctx
    from minisgl_amd.layers import MoELayer

    reset_global_ctx()
    with pytest.raises(RuntimeError, match="context"):
        MoELayer(4, 2, 16, 8).forward(torch.zeros(1, 16), torch.zeros(1, 4))


def test_backend_requires_scales():
    from minisgl_amd.moe import create_moe_backend

    with pytest.raises(ValueError, match="scale"):
        create_moe_backend("fused_w8a8").forward(torch.zeros(1, 16), torch.zeros(4, 16, 16), torch.zeros(4, 16, 8),
                                                 torch.zeros(1, 4), 2, True)


def test_default_tiling_of_the_benchmark_shapes(lib):
    """The tiling the library picks for each Qwen3-14B benchmark shape (the
    time model plus the split-K rules, planned for 256 CUs without a GPU):
    decode cores up to 8 rows (the shared token ring for the wide gate_up at
    8 rows), in-block split-K for qkv / o_proj at 64 and 512 rows, the
    shared token ring for gate_up and the 64x128 ring for the deep down at
    64 rows, and above the 256x256 ring (its weight stages a stage ahead)
    or, where it fills the last wave of the CUs better (N = 5120, qkv at
    8192 rows), the 256x320 ring."""
    t3 = "tile3_gemm_kernel<{}, {}, 128, {}, {}, {}>"
    sq, wide = t3.format(256, 256, 2, 4, 2), t3.format(256, 320, 2, 4, 2)
    ks64, ks512 = "ksplit_gemm_kernel<64, 32, 8, 1, 1, 2, 3>", "ksplit_gemm_kernel<128, 128, 2, 2, 2, 2, 3>"
    r64 = t3.format(64, 128, 1, 4, 4)
    expect = {
        (5120, 7168): [ks64, ks512, sq, wide],
        (5120, 5120): [ks64, ks512, wide, wide],
        (5120, 34816): ["decode_sx_gemm_kernel", wide, sq, sq],
        (17408, 5120): [r64, sq, wide, wide],
    }
    for (K, N), names in expect.items():
        assert lib.mw8_gemm_kernel_name(1, N, K) == b"decode3_gemm_kernel", (1, N, K)
        # 8 tokens: the shared token ring for the wide gate_up, decode3 otherwise
        want8 = b"decode_sx_gemm_kernel" if N >= 16384 else b"decode3_gemm_kernel"
        assert lib.mw8_gemm_kernel_name(8, N, K) == want8, (8, N, K)
        for M, name in zip((64, 512, 4096, 8192), names):
            assert lib.mw8_gemm_kernel_name(M, N, K).decode() == name, (M, N, K)


def test_mid_m_tiling_fills_one_wave(lib):
    """Between 65 and 768 rows qkv / o_proj take the smallest split-K tile
    whose fewest column ranges fit one wave of 256 CUs, and the ring when
    none does (qkv at 640 / 768 rows)."""
    k64 = "ksplit_gemm_kernel<64, 64, 8, 1, 1, 1, 4>"
    k128x64 = "ksplit_gemm_kernel<128, 64, 4, 2, 1, 2, 3>"
    k128 = "ksplit_gemm_kernel<128, 128, 2, 2, 2, 2, 3>"
    ring = "tile3_gemm_kernel<256, 128, 128, 4, 2, 3>"
    expect = {
        7168: {96: k64, 128: k64, 192: k128x64, 256: k128x64, 320: k128, 384: k128, 512: k128,
               640: ring, 768: ring},
        5120: {96: k64, 128: k64, 192: k64, 256: k128x64, 384: k128x64, 512: k128, 768: k128},
    }
    for N, by_m in expect.items():
        for M, name in by_m.items():
            assert lib.mw8_gemm_kernel_name(M, N, 5120).decode() == name, (M, N)
