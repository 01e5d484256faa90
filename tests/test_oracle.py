"""CPU tests that pin the oracle (oracle/w8a8.py) to independent facts:
exact-rational golden vectors (tests/golden/make_golden.py), the
reference's docstring known answer for moe_align_block_size, torch library
routines (round-half-even, _int_mm, bf16 cast, softmax/top-k, silu),
brute force on tiny inputs, and closed forms.  Each "planted" test swaps a
plausible mistake into the oracle (on the CPU) and shows a check catches it.
"""

import os

import numpy as np
import pytest
import torch

from oracle import w8a8 as orc

GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "w8a8_golden.npz"))


def _bf16(x: np.ndarray) -> np.ndarray:
    return torch.from_numpy(np.ascontiguousarray(x, np.float32)).to(torch.bfloat16).float().numpy()


# ------------------------------------------------------------------ quantizer
def test_quant_golden_exact():
    q, s = orc.quant_per_token(GOLDEN["quant_x"])
    np.testing.assert_array_equal(q, GOLDEN["quant_q"])
    np.testing.assert_array_equal(s.view(np.uint32), GOLDEN["quant_s"].view(np.uint32))


def test_quant_ties_round_half_even():
    q, s = orc.quant_per_token(GOLDEN["quant_x"][:1])
    assert s[0] == 1.0
    assert q[0, :6].tolist() == [127, 2, 0, 126, 4, -2]


def test_quant_zero_single_outlier_rows():
    q, s = orc.quant_per_token(GOLDEN["quant_x"][1:4])
    assert q[0, 3] == -127 and s[0] == np.float32(3.0) / np.float32(127.0)
    assert s[1] == 0 and not q[1].any()
    assert q[2, 0] == 127 and abs(int(q[2, 3])) <= 1


def test_quant_matches_torch_round_seeded():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(64, 1024, generator=g)
    x[torch.rand(64, 1024, generator=g) < 1e-3] *= 20
    x = x.to(torch.bfloat16).float()
    s_t = x.abs().amax(1) / 127.0
    q_t = torch.clamp(torch.round(x / s_t[:, None]), -127, 127).to(torch.int8)
    q, s = orc.quant_per_token(x.numpy())
    np.testing.assert_array_equal(s, s_t.numpy())
    np.testing.assert_array_equal(q, q_t.numpy())


def test_planted_round_half_away_is_caught(monkeypatch):
    monkeypatch.setattr(orc.np, "rint", lambda t: np.floor(t + 0.5))
    q, _ = orc.quant_per_token(GOLDEN["quant_x"])
    assert not np.array_equal(q, GOLDEN["quant_q"])


def test_planted_reciprocal_multiply_is_caught():
    """x * (1/s) instead of x / s changes some integers (the reason the
    kernel corrects its reciprocal product with an FMA residual)."""
    x = torch.randn(2048, 512, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).float().numpy()
    q, s = orc.quant_per_token(x)
    r = (np.float32(1.0) / s).astype(np.float32)
    q_bad = np.clip(np.rint((x * r[:, None]).astype(np.float32)), -127, 127).astype(np.int8)
    assert not np.array_equal(q, q_bad)


def test_quant_kernel_division_exhaustive(tmp_path):
    """Compile the kernel's per-element quantizer math (mw8_common.h) for the
    host and check it against IEEE division for every bf16 input."""
    import shutil
    import subprocess

    if shutil.which("g++") is None:
        pytest.skip("g++ not available")
    root = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
    exe = tmp_path / "qmc"
    subprocess.run(
        ["g++", "-O2", "-std=c++17", "-ffp-contract=off",
         "-I", os.path.join(root, "mini-sglang-fork_amd", "csrc"),
         os.path.join(root, "tests", "native", "quant_math_check.cpp"), "-o", str(exe)],
        check=True,
    )
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0, out.stdout + out.stderr
    assert "mismatches=0 quotient_mismatches=0" in out.stdout


# ------------------------------------------------------------------ GEMM
def test_gemm_golden_exact():
    acc = orc.gemm_i32(GOLDEN["quant_q"], GOLDEN["gemm_w"])
    np.testing.assert_array_equal(acc, GOLDEN["gemm_acc"])


def test_gemm_matches_torch_int_mm():
    g = torch.Generator().manual_seed(1)
    a = torch.randint(-127, 128, (48, 1024), generator=g, dtype=torch.int8)
    w = torch.randint(-127, 128, (96, 1024), generator=g, dtype=torch.int8)
    ref = torch._int_mm(a, w.t().contiguous())
    np.testing.assert_array_equal(orc.gemm_i32(a.numpy(), w.numpy()), ref.numpy())


def test_gemm_extremes_closed_form():
    K = 25600
    a = np.full((2, K), 127, np.int8)
    w = np.full((3, K), -127, np.int8)
    assert (orc.gemm_i32(a, w) == -K * 127 * 127).all()


def test_gemm_brute_force_tiny():
    rng = np.random.default_rng(2)
    a = rng.integers(-127, 128, (3, 128), dtype=np.int64).astype(np.int8)
    w = rng.integers(-127, 128, (5, 128), dtype=np.int64).astype(np.int8)
    ref = [[sum(int(x) * int(y) for x, y in zip(a[m], w[n])) for n in range(5)] for m in range(3)]
    np.testing.assert_array_equal(orc.gemm_i32(a, w), np.array(ref))


def test_planted_dropped_k_term_is_caught(monkeypatch):
    real = orc.gemm_i32

    def dropped(a, w):
        return real(a[:, :-1], w[:, :-1])

    monkeypatch.setattr(orc, "gemm_i32", dropped)
    assert not np.array_equal(orc.gemm_i32(GOLDEN["quant_q"], GOLDEN["gemm_w"]), GOLDEN["gemm_acc"])


# ------------------------------------------------------------------ epilogue
def test_epilogue_golden_exact():
    y = orc.epilogue(GOLDEN["gemm_acc"], GOLDEN["quant_s"], GOLDEN["gemm_sw"])
    np.testing.assert_array_equal(y.view(np.uint32), GOLDEN["gemm_y"].view(np.uint32))


def test_epilogue_matches_torch_bf16_cast():
    g = torch.Generator().manual_seed(4)
    acc = torch.randint(-(2**28), 2**28, (64, 96), generator=g, dtype=torch.int32)
    sa = torch.rand(64, generator=g) * 1e-2
    sw = torch.rand(96, generator=g) * 1e-2
    b = torch.randn(96, generator=g).to(torch.bfloat16)
    ref = ((acc.float() * sa[:, None]) * sw[None, :] + b.float()[None, :]).to(torch.bfloat16).float()
    y = orc.epilogue(acc.numpy(), sa.numpy(), sw.numpy(), b.float().numpy())
    np.testing.assert_array_equal(y, ref.numpy())


def test_bf16_round_ties_even():
    x = np.array([1 + 2**-8, 1 + 3 * 2**-8, -(1 + 2**-8), 3.0, 1 + 2**-9], np.float32)
    np.testing.assert_array_equal(orc.bf16_round(x), _bf16(x))
    assert orc.bf16_round(x)[0] == 1.0 and orc.bf16_round(x)[1] == 1 + 2**-6


def test_planted_reassociated_epilogue_is_caught():
    """acc * (sa * sw) (a re-associated product) differs from the oracle's
    ((acc * sa) * sw) in fp32; after bf16 narrowing the difference survives
    on a small fraction of elements, so a large sample shows it."""
    g = torch.Generator().manual_seed(5)
    acc = torch.randint(-(2**28), 2**28, (1024, 1024), generator=g, dtype=torch.int32).numpy()
    sa = (torch.rand(1024, generator=g) * 1e-2).numpy()
    sw = (torch.rand(1024, generator=g) * 1e-2).numpy()
    good = orc.epilogue(acc, sa, sw)
    bad = orc.bf16_round(acc.astype(np.float32) * (sa[:, None] * sw[None, :]).astype(np.float32))
    assert 0 < (good != bad).sum() < good.size // 100


def test_planted_swapped_scales_is_caught(monkeypatch):
    real = orc.epilogue
    def swapped(acc, sa, sw, **kw):  # row and column scales exchanged (cycled to fit)
        return real(acc, np.resize(sw, acc.shape[0]), np.resize(sa, acc.shape[1]), **kw)

    monkeypatch.setattr(orc, "epilogue", swapped)
    y = orc.epilogue(GOLDEN["gemm_acc"], GOLDEN["quant_s"], GOLDEN["gemm_sw"])
    assert not np.array_equal(y, GOLDEN["gemm_y"])


# ------------------------------------------------------------------ routing
def test_topk_matches_torch():
    """Selected weights equal torch.softmax + torch.topk + the two
    renormalisations; ids form a valid top-k (every selected probability >=
    every unselected one).  Ties (bf16 logits repeat) are broken toward the
    lower expert index; the reference's sgl_kernel tie order is not
    available (parity unpinned there)."""
    g = torch.Generator().manual_seed(6)
    logits = torch.randn(64, 128, generator=g).to(torch.bfloat16).float()
    p = torch.softmax(logits, -1)
    tw, _ = torch.topk(p, 8, -1)
    tw = tw / tw.sum(-1, keepdim=True)
    tw = tw / (tw.sum(-1, keepdim=True) + 1e-8)
    w, ids = orc.topk_softmax(logits.numpy(), 8, True)
    np.testing.assert_allclose(w, tw.numpy(), rtol=1e-6, atol=1e-7)
    np.testing.assert_allclose(w.sum(-1), 1.0, rtol=1e-6)
    pn = p.numpy()
    for r in range(pn.shape[0]):
        sel = pn[r, ids[r]]
        rest = np.delete(pn[r], ids[r])
        assert sel.min() >= rest.max()
        assert len(set(ids[r].tolist())) == 8
        for a in range(7):  # equal probabilities: lower index first
            if sel[a] == sel[a + 1]:
                assert ids[r, a] < ids[r, a + 1]


def test_topk_no_renorm_keeps_softmax_mass():
    logits = np.random.default_rng(7).standard_normal((5, 64)).astype(np.float32)
    w, _ = orc.topk_softmax(logits, 2, False)
    assert (w.sum(-1) < 1).all()


# ------------------------------------------------------------------ alignment
def test_align_docstring_known_answer():
    s, e, n = orc.moe_align_block_size(GOLDEN["align_topk_ids"], 4, 4)
    assert n == int(GOLDEN["align_num_post_pad"][0])
    np.testing.assert_array_equal(s[:n], GOLDEN["align_sorted_ids"])
    np.testing.assert_array_equal(e[: n // 4], GOLDEN["align_expert_ids"])
    assert s.size == 12 + 5 * 3  # numel + (E + 1) * (B - 1), python/minisgl/moe/fused.py:73


@pytest.mark.parametrize("M,k,E,B", [(16, 8, 128, 16), (256, 8, 128, 64), (37, 3, 7, 4), (1, 1, 1, 16)])
def test_align_invariants(M, k, E, B):
    ids = np.random.default_rng(M * E).integers(0, E, (M, k)).astype(np.int32)
    s, e, n = orc.moe_align_block_size(ids, B, E)
    flat = ids.reshape(-1)
    numel = flat.size
    assert s.size == numel + (E + 1) * (B - 1)
    assert e.size == -(-s.size // B)
    counts = np.bincount(flat, minlength=E + 1)
    assert n == sum(-(-c // B) * B for c in counts)
    assert n % B == 0 and (s[n:] == numel).all() and (e[n // B:] == -1).all()
    seen = []
    for b in range(n // B):
        blk = s[b * B:(b + 1) * B]
        real = blk[blk < numel]
        assert (flat[real] == e[b]).all()
        seen.extend(real.tolist())
    assert sorted(seen) == list(range(numel))  # every pair exactly once


def test_planted_unpadded_alignment_is_caught(monkeypatch):
    real = orc.moe_align_block_size
    monkeypatch.setattr(orc, "moe_align_block_size", lambda ids, B, E: real(ids, 1, E))
    s, _, n = orc.moe_align_block_size(GOLDEN["align_topk_ids"], 4, 4)
    assert n != 16


def test_block_size_regimes():
    # python/minisgl/moe/fused.py:106-113: M <= E -> 16-row blocks, else 64
    assert orc.moe_block_size(16, 128) == 16 and orc.moe_block_size(128, 128) == 16
    assert orc.moe_block_size(129, 128) == 64


# ------------------------------------------------------------------ activation
def test_silu_and_mul_matches_torch():
    g = torch.Generator().manual_seed(8)
    x = torch.randn(16, 1536, generator=g).to(torch.bfloat16).float()
    d = 768
    ref = (torch.nn.functional.silu(x[:, :d]) * x[:, d:]).to(torch.bfloat16).float().numpy()
    got = orc.silu_and_mul(x.numpy())
    # exp implementations may differ by an ulp: allow one bf16 ulp
    assert np.abs(got - ref).max() <= np.abs(ref).max() * 2**-7
    assert (got == ref).mean() > 0.99


def test_gelu_and_mul_matches_torch():
    g = torch.Generator().manual_seed(9)
    x = torch.randn(8, 64, generator=g).to(torch.bfloat16).float()
    ref = (torch.nn.functional.gelu(x[:, :32]) * x[:, 32:]).to(torch.bfloat16).float().numpy()
    got = orc.gelu_and_mul(x.numpy())
    assert (got == ref).mean() > 0.98 and np.abs(got - ref).max() <= np.abs(ref).max() * 2**-7


def test_act_gate_first():
    x = np.zeros((1, 4), np.float32)
    x[0, :2] = [100.0, 0.0]
    x[0, 2:] = [2.0, 5.0]
    np.testing.assert_allclose(orc.silu_and_mul(x)[0], [200.0, 0.0])


# ------------------------------------------------------------------ slot sum
def test_sum_reduce_sequential_fp32_order():
    x = np.array([[[2.0**24] * 8, [1.0] * 8, [-(2.0**24)] * 8]], np.float32)
    assert (orc.moe_sum_reduce(x) == 0).all()  # sequential fp32: (2^24 + 1) rounds to 2^24
    assert x.astype(np.float64).sum(1).max() == 1.0


def test_sum_reduce_small_integers_exact():
    x = np.random.default_rng(10).integers(-50, 50, (5, 8, 64)).astype(np.float32)
    np.testing.assert_array_equal(orc.moe_sum_reduce(x), x.sum(1))


# ------------------------------------------------------------------ whole layer
def test_fused_moe_brute_force_tiny():
    rng = np.random.default_rng(11)
    M, H, I, E, k = 5, 64, 32, 4, 2
    hidden = _bf16(rng.standard_normal((M, H)))
    w1 = rng.integers(-127, 128, (E, 2 * I, H)).astype(np.int8)
    w2 = rng.integers(-127, 128, (E, H, I)).astype(np.int8)
    s1 = (rng.random((E, 2 * I)) * 1e-2).astype(np.float32)
    s2 = (rng.random((E, H)) * 1e-2).astype(np.float32)
    logits = _bf16(rng.standard_normal((M, E)))
    out = orc.fused_moe_w8a8(hidden, w1, s1, w2, s2, logits, k)
    tw, ids = orc.topk_softmax(logits, k, True)
    q_h, s_h = orc.quant_per_token(hidden)
    ref = np.zeros((M, H), np.float32)
    rows = []
    for t in range(M):
        per_slot = []
        for i in range(k):
            e = ids[t, i]
            a1 = [int(np.dot(q_h[t].astype(np.int64), w1[e, n].astype(np.int64))) for n in range(2 * I)]
            c1 = orc.epilogue(np.array([a1], np.int32), s_h[t:t + 1], s1[e])
            act = orc.silu_and_mul(c1)
            q_a, s_a = orc.quant_per_token(act)
            a2 = [int(np.dot(q_a[0].astype(np.int64), w2[e, n].astype(np.int64))) for n in range(H)]
            per_slot.append(orc.epilogue(np.array([a2], np.int32), s_a, s2[e], routed=tw[t, i:i + 1])[0])
        rows.append(per_slot)
    ref = orc.moe_sum_reduce(np.array(rows, np.float32))
    np.testing.assert_array_equal(out, ref)
    # and the W8A8 layer tracks the float MoE (quantization error only)
    f = np.zeros((M, H))
    for t in range(M):
        for i in range(k):
            e = ids[t, i]
            g1 = (w1[e].astype(np.float64) * s1[e][:, None]) @ hidden[t]
            a = g1[:I] / (1 + np.exp(-g1[:I])) * g1[I:]
            f[t] += tw[t, i] * ((w2[e].astype(np.float64) * s2[e][:, None]) @ a)
    assert np.linalg.norm(out - f) / np.linalg.norm(f) < 0.05


# ------------------------------------------------------- RMSNorm + requant
def _rms_torch64(h, w, eps):
    """Independent restatement in torch float64 (no fp32 rounding steps)."""
    h64 = torch.from_numpy(np.asarray(h, np.float64))
    w64 = torch.from_numpy(np.asarray(w, np.float64))
    r = torch.rsqrt((h64 * h64).mean(dim=1, keepdim=True) + eps)
    return (h64 * r * w64).numpy()


def test_rmsnorm_closed_forms():
    """Constant rows give r exactly: c = 2, eps = 0 -> r = 1/2 and y = w;
    eps = 12 -> r = 1/sqrt(16) = 1/4 and y = w / 2."""
    H = 64
    w = _bf16(np.linspace(-3, 3, H).astype(np.float32))
    x = np.full((2, H), 2.0, np.float32)
    _, _, y0, _ = orc.rmsnorm_quant(x, w, 0.0)
    np.testing.assert_array_equal(y0, np.broadcast_to(w, (2, H)))
    _, _, y1, _ = orc.rmsnorm_quant(x, w, 12.0)
    np.testing.assert_array_equal(y1, np.broadcast_to(_bf16(w / 2), (2, H)))


def test_rmsnorm_matches_torch_float64():
    """Seeded rows with outliers: the fp32 closed form agrees with a torch
    float64 RMSNorm to bf16 rounding, and the sum of squares it uses is the
    exact rational one."""
    from fractions import Fraction

    gen = torch.Generator().manual_seed(5)
    x = torch.randn(16, 2048, generator=gen)
    x[torch.rand(16, 2048, generator=gen) < 1e-3] *= 20
    x = x.to(torch.bfloat16).float().numpy()
    w = (torch.rand(2048, generator=gen) + 0.5).to(torch.bfloat16).float().numpy()
    q, s, y, h = orc.rmsnorm_quant(x, w, 1e-6)
    ref = _rms_torch64(x, w, 1e-6)
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-30)) <= 2.0 ** -8 + 1e-6
    exact = sum(Fraction(float(v)) ** 2 for v in x[3])
    assert float(exact) == float((x[3].astype(np.float64) ** 2).sum())
    q2, s2 = orc.quant_per_token(y)
    np.testing.assert_array_equal(q, q2)
    np.testing.assert_array_equal(s, s2)


def test_rmsnorm_residual_add_matches_torch_bf16():
    gen = torch.Generator().manual_seed(6)
    x = torch.randn(4, 512, generator=gen).to(torch.bfloat16)
    res = torch.randn(4, 512, generator=gen).to(torch.bfloat16)
    w = torch.ones(512).to(torch.bfloat16)
    _, _, y, h = orc.rmsnorm_quant(x.float().numpy(), w.float().numpy(), 1e-5, residual=res.float().numpy())
    np.testing.assert_array_equal(h, (x + res).float().numpy())  # torch: fp32 add, RNE to bf16
    ref = _rms_torch64(h, w.float().numpy(), 1e-5)
    assert np.max(np.abs(y - ref) / (np.abs(ref) + 1e-30)) <= 2.0 ** -8 + 1e-6


@pytest.mark.parametrize("mistake", ["eps_outside_sqrt", "mean_over_h_minus_1", "no_weight"])
def test_planted_rmsnorm_mistakes_are_caught(mistake):
    """Plant a plausible mistake into a copy of the closed form: the float64
    torch cross-check catches each (H = 16: a mean over H - 1 is then off by
    3%, beyond bf16 rounding)."""
    H = 16
    gen = torch.Generator().manual_seed(7)
    x = torch.randn(8, H, generator=gen).to(torch.bfloat16).float().numpy()
    w = (torch.rand(H, generator=gen) + 0.5).to(torch.bfloat16).float().numpy()
    eps = 0.5  # large enough that misplacing it matters

    def planted(xx):
        ss = (xx.astype(np.float64) ** 2).sum(axis=1)
        div = H - 1 if mistake == "mean_over_h_minus_1" else H
        ms = (ss / div).astype(np.float32)
        if mistake == "eps_outside_sqrt":
            r = (np.float32(1) / np.sqrt(ms, dtype=np.float32) + np.float32(eps)).astype(np.float32)
        else:
            r = (np.float32(1) / np.sqrt(ms + np.float32(eps), dtype=np.float32)).astype(np.float32)
        ww = np.ones_like(w) if mistake == "no_weight" else w
        return orc.bf16_round((xx * r[:, None]).astype(np.float32) * ww)

    ref = _rms_torch64(x, w, eps)
    good = orc.rmsnorm_quant(x, w, eps)[2]
    assert np.max(np.abs(good - ref) / (np.abs(ref) + 1e-30)) <= 2.0 ** -8 + 1e-6
    bad = planted(x)
    assert np.max(np.abs(bad - ref) / (np.abs(ref) + 1e-30)) > 2.0 ** -6
