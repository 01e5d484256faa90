"""CPU oracle for the W8A8 int8 linear and fused-MoE path.

TEST INFRASTRUCTURE ONLY. This module is the checker that the HIP kernels are
compared against. Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import it; the product path under
``mini-sglang-fork_amd/`` never does, and fails loudly when its HIP library is
missing instead of falling back here.

Everything is plain numpy (float32 / int arithmetic with IEEE round-to-nearest
semantics).  bf16 tensors are represented as float32 arrays whose values are
exactly representable in bf16; :func:`bf16_round` performs the
round-to-nearest-even narrowing.

The reference (mini-sglang) has no int8 code: its linear slot is a bf16
``F.linear`` (python/minisgl/layers/linear.py:31-32) and its MoE slot a bf16
Triton grouped GEMM (python/minisgl/moe/fused.py:127-227).  The W8A8
arithmetic is therefore defined here by closed forms, while layouts, routing,
alignment and buffer flow follow the reference line by line (citations on
each function).

Pinning (what fixes each function independently of its own formula; the
checks live in tests/test_oracle.py):

* quant_per_token   -- hand-built tie rows (round-half-even), zero / single
                       value / outlier rows, torch.round cross-check.
* gemm_i32          -- torch._int_mm (independent int8 GEMM), extreme-value
                       closed form K*127*127, brute force on tiny inputs.
* epilogue          -- torch bf16 cast (independent RNE narrowing), exact
                       small-integer cases.
* topk_softmax      -- torch.softmax + torch.topk; weights sum to one.
* moe_align         -- the reference docstring known-answer vector
                       (python/minisgl/moe/fused.py:56-69) + invariants.
* silu_and_mul      -- torch.nn.functional.silu (tolerance: exp differs by
                       <= 1 ulp between libraries).
* moe_sum_reduce    -- a rounding-order case whose sequential fp32 result
                       differs from the exact sum; small-integer exact sums.
* fused_moe_w8a8    -- brute-force per-(token, slot) loop on tiny shapes.
* rmsnorm_quant     -- exact rational sum of squares (fractions), a torch
                       fp64 RMSNorm cross-check, the residual add against
                       torch's bf16 add, and planted mistakes (eps outside
                       the square root, mean over H-1, no weight).

Top-k tie-breaking and the order of pairs inside one expert segment are
internals of the third-party ``sgl_kernel`` (>=0.3.17.post1, not vendored):
parity unpinned there.  Segment order does not change any result (GEMM rows
are independent); ties have probability ~0 for continuous logits.
"""

from __future__ import annotations

from typing import Optional, Tuple

import numpy as np

__all__ = [
    "bf16_round",
    "bf16_bits",
    "from_bf16_bits",
    "quant_per_token",
    "gemm_i32",
    "epilogue",
    "linear_w8a8",
    "topk_softmax",
    "moe_align_block_size",
    "moe_block_size",
    "silu_and_mul",
    "gelu_and_mul",
    "act_and_mul_quant",
    "moe_sum_reduce",
    "grouped_gemm_w8a8",
    "fused_moe_w8a8",
    "rmsnorm_quant",
]

_F32 = np.float32


# --------------------------------------------------------------------------
# bf16 helpers
# --------------------------------------------------------------------------
def bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 bit pattern (uint16), round-to-nearest-even.  Finite inputs."""
    u = np.ascontiguousarray(x, dtype=_F32).view(np.uint32).astype(np.uint64)
    u = u + 0x7FFF + ((u >> 16) & 1)
    return (u >> 16).astype(np.uint16)


def from_bf16_bits(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b, dtype=np.uint16).astype(np.uint32) << 16).view(_F32)


def bf16_round(x: np.ndarray) -> np.ndarray:
    """Round fp32 values to bf16 precision (RNE) and return them as fp32."""
    return from_bf16_bits(bf16_bits(x))


# --------------------------------------------------------------------------
# A3: per-token dynamic quantizer (no reference function; inserted before
# F.linear at python/minisgl/layers/linear.py:32 and before both grouped
# GEMMs at python/minisgl/moe/fused.py:192,208)
# --------------------------------------------------------------------------
def quant_per_token(x: np.ndarray) -> Tuple[np.ndarray, np.ndarray]:
    """``s = amax/127`` (fp32 IEEE division), ``q = clamp(rint(x/s), -127, 127)``.

    ``x`` is float32 [M, K] holding bf16 values.  A row of zeros gives
    ``s = 0`` and ``q = 0``.  Returns (q int8 [M, K], s float32 [M]).
    """
    x = np.asarray(x, dtype=_F32)
    assert x.ndim == 2
    M, K = x.shape
    amax = np.abs(x).max(axis=1) if K > 0 else np.zeros(M, _F32)
    s = (amax.astype(_F32) / _F32(127.0)).astype(_F32)
    q = np.zeros((M, K), dtype=np.int8)
    nz = s > 0
    if nz.any():
        t = x[nz] / s[nz, None]  # float32 / float32: one IEEE RN division
        assert t.dtype == _F32
        q[nz] = np.clip(np.rint(t), -127, 127).astype(np.int8)
    return q, s


# --------------------------------------------------------------------------
# A4: exact int32 GEMM + fp32 epilogue (replaces F.linear,
# python/minisgl/layers/linear.py:31-32; weight layout [N, K] from :28)
# --------------------------------------------------------------------------
def gemm_i32(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """``acc[m, n] = sum_k a[m, k] * w[n, k]`` exactly, as int32.

    Computed in float64, which is exact because every partial sum is an
    integer below 2**53 (|acc| <= K * 127 * 128).
    """
    a = np.asarray(a)
    w = np.asarray(w)
    assert a.dtype == np.int8 and w.dtype == np.int8
    assert a.ndim == 2 and w.ndim == 2 and a.shape[1] == w.shape[1]
    assert a.shape[1] * 128 * 128 < 2**53
    acc = a.astype(np.float64) @ w.astype(np.float64).T
    acc = acc.astype(np.int64)
    assert np.all(np.abs(acc) < 2**31), "int32 accumulator overflow"
    return acc.astype(np.int32)


def epilogue(
    acc: np.ndarray,
    s_a: np.ndarray,
    s_w: np.ndarray,
    bias: Optional[np.ndarray] = None,
    routed: Optional[np.ndarray] = None,
) -> np.ndarray:
    """``bf16(((float(acc) * s_a[m]) * s_w[n]) [+ bias[n]] [* routed[m]])``.

    Each operation is one fp32 rounding (no fused multiply-add).  The routed
    weight multiply follows the scales and precedes the bf16 cast, the order
    of python/minisgl/kernel/triton/fused_moe.py:183-187.  Returns fp32 values
    on the bf16 grid.
    """
    t = np.asarray(acc, dtype=np.int32).astype(_F32)
    t = t * np.asarray(s_a, dtype=_F32)[:, None]
    t = t * np.asarray(s_w, dtype=_F32)[None, :]
    if bias is not None:
        t = t + np.asarray(bias, dtype=_F32)[None, :]
    if routed is not None:
        t = t * np.asarray(routed, dtype=_F32)[:, None]
    assert t.dtype == _F32
    return bf16_round(t)


def linear_w8a8(
    x: np.ndarray, w: np.ndarray, s_w: np.ndarray, bias: Optional[np.ndarray] = None
) -> Tuple[np.ndarray, np.ndarray, np.ndarray, np.ndarray]:
    """Whole W8A8 linear forward: quant -> int GEMM -> epilogue.

    Returns (y, q, s_a, acc) so that every stage can be compared.
    """
    q, s_a = quant_per_token(x)
    acc = gemm_i32(q, w)
    return epilogue(acc, s_a, s_w, bias), q, s_a, acc


# --------------------------------------------------------------------------
# A6: router top-k (python/minisgl/moe/fused.py:9-28)
# --------------------------------------------------------------------------
def topk_softmax(
    logits: np.ndarray, topk: int, renormalize: bool
) -> Tuple[np.ndarray, np.ndarray]:
    """fp32 softmax over experts, top-k (larger index loses ties), optional
    renormalisation twice: ``w/sum(w)`` inside the top-k op and then
    ``w/(sum(w)+1e-8)`` (python/minisgl/moe/fused.py:22-24)."""
    lg = np.asarray(logits, dtype=_F32)
    mx = lg.max(axis=1, keepdims=True)
    e = np.exp(lg - mx).astype(_F32)
    p = (e / e.sum(axis=1, keepdims=True, dtype=_F32)).astype(_F32)
    order = np.argsort(-p, axis=1, kind="stable")[:, :topk]
    ids = order.astype(np.int32)
    w = np.take_along_axis(p, order, axis=1).astype(_F32)
    if renormalize:
        w = (w / w.sum(axis=1, keepdims=True, dtype=_F32)).astype(_F32)
        w = (w / (w.sum(axis=1, keepdims=True, dtype=_F32) + _F32(1e-8))).astype(_F32)
    return w, ids


# --------------------------------------------------------------------------
# A7 / A8: alignment and tile regime (python/minisgl/moe/fused.py:31-124)
# --------------------------------------------------------------------------
def moe_block_size(M: int, E: int) -> int:
    """BLOCK_SIZE_M of the reference's default config: 16 when M <= E, else 64
    (python/minisgl/moe/fused.py:100-113)."""
    return 16 if M <= E else 64


def moe_align_block_size(
    topk_ids: np.ndarray, block_size: int, num_experts: int
) -> Tuple[np.ndarray, np.ndarray, int]:
    """Group flat (token, slot) indices by expert, pad each group to a multiple
    of ``block_size`` with the sentinel ``numel``.

    Mirrors python/minisgl/moe/fused.py:31-89: ``num_experts + 1`` expert slots
    (:81), buffer sizes from :73-76, padding with the sentinel everywhere
    (:87).  Inside a segment pairs are in ascending flat order (the order of
    the docstring example, :56-69).  Blocks past the used range get expert
    id -1.  Returns (sorted_ids, expert_ids, num_tokens_post_pad).
    """
    ids = np.asarray(topk_ids).astype(np.int64).reshape(-1)
    numel = ids.size
    slots = num_experts + 1
    max_padded = numel + slots * (block_size - 1)
    max_blocks = -(-max_padded // block_size)
    sorted_ids = np.full(max_padded, numel, dtype=np.int32)
    expert_ids = np.full(max_blocks, -1, dtype=np.int32)
    pos = 0
    for e in range(slots):
        members = np.nonzero(ids == e)[0]
        cnt = members.size
        if cnt == 0:
            continue
        padded = -(-cnt // block_size) * block_size
        sorted_ids[pos : pos + cnt] = members
        expert_ids[pos // block_size : (pos + padded) // block_size] = e
        pos += padded
    return sorted_ids, expert_ids, pos


# --------------------------------------------------------------------------
# A11: activation (python/minisgl/layers/activation.py:9-18, gate first)
# --------------------------------------------------------------------------
def silu_and_mul(x: np.ndarray) -> np.ndarray:
    """``bf16(silu(g) * u)`` with ``silu(g) = g / (1 + exp(-g))`` in fp32."""
    x = np.asarray(x, dtype=_F32)
    d = x.shape[1] // 2
    g, u = x[:, :d], x[:, d:]
    with np.errstate(over="ignore"):
        act = (g / (_F32(1.0) + np.exp(-g))).astype(_F32)
    return bf16_round((act * u).astype(_F32))


def gelu_and_mul(x: np.ndarray) -> np.ndarray:
    """``bf16(gelu(g) * u)`` with the erf form ``0.5 g (1 + erf(g/sqrt(2)))``."""
    from math import erf, sqrt

    x = np.asarray(x, dtype=_F32)
    d = x.shape[1] // 2
    g, u = x[:, :d].astype(np.float64), x[:, d:]
    verf = np.vectorize(erf)
    act = (0.5 * g * (1.0 + verf(g / sqrt(2.0)))).astype(_F32)
    return bf16_round((act * u).astype(_F32))


def act_and_mul_quant(x: np.ndarray, activation: str = "silu"):
    """Fused activation + requant: returns (q int8, s fp32, act bf16-as-fp32)."""
    act = silu_and_mul(x) if activation == "silu" else gelu_and_mul(x)
    q, s = quant_per_token(act)
    return q, s, act


# --------------------------------------------------------------------------
# A12: top-k sum (python/minisgl/kernel/triton/fused_moe.py:5-47)
# --------------------------------------------------------------------------
def moe_sum_reduce(x: np.ndarray) -> np.ndarray:
    """``out[t] = bf16(sum_i x[t, i])`` summed in fp32 in slot order (:36-47)."""
    x = np.asarray(x, dtype=_F32)
    acc = np.zeros((x.shape[0], x.shape[2]), dtype=_F32)
    for i in range(x.shape[1]):
        acc = (acc + x[:, i, :]).astype(_F32)
    return bf16_round(acc)


# --------------------------------------------------------------------------
# A10: grouped GEMM over expert segments
# (python/minisgl/kernel/triton/fused_moe.py:50-193)
# --------------------------------------------------------------------------
def grouped_gemm_w8a8(
    q: np.ndarray,
    s_a: np.ndarray,
    w: np.ndarray,
    s_w: np.ndarray,
    topk_ids: np.ndarray,
    top_k: int,
    routed: Optional[np.ndarray] = None,
    return_acc: bool = False,
):
    """One grouped GEMM.  Row ``p`` of the output (a flat (token, slot) pair)
    is ``epilogue(q[p // top_k] . w[e_p]^T, s_a[p // top_k], s_w[e_p])``
    optionally times ``routed[p]``; A rows are addressed ``sorted_id //
    top_k`` (:142), the output row is the pair index (:190-193), the routed
    weight is indexed by the pair (:184).

    ``q`` int8 [T, K], ``w`` int8 [E, N, K], ``s_w`` fp32 [E, N],
    ``topk_ids`` [T / top_k * top_k...] flat pair -> expert.
    Returns bf16-as-fp32 [P, N] (and int32 acc [P, N] if requested).
    """
    ids = np.asarray(topk_ids).reshape(-1).astype(np.int64)
    P = ids.size
    N = w.shape[1]
    out = np.zeros((P, N), dtype=_F32)
    acc_all = np.zeros((P, N), dtype=np.int32) if return_acc else None
    for e in np.unique(ids):
        rows = np.nonzero(ids == e)[0]
        tok = rows // top_k
        acc = gemm_i32(q[tok], w[e])
        r = None if routed is None else np.asarray(routed, _F32).reshape(-1)[rows]
        out[rows] = epilogue(acc, np.asarray(s_a)[tok], s_w[e], routed=r)
        if return_acc:
            acc_all[rows] = acc
    return (out, acc_all) if return_acc else out


def fused_moe_w8a8(
    hidden: np.ndarray,
    w1: np.ndarray,
    s_w1: np.ndarray,
    w2: np.ndarray,
    s_w2: np.ndarray,
    logits: np.ndarray,
    topk: int,
    renormalize: bool = True,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
    stages: bool = False,
):
    """The whole W8A8 fused-MoE layer, following fused_experts_impl
    (python/minisgl/moe/fused.py:127-227): route, quantize hidden once,
    GEMM1 (routed weight only if ``apply_router_weight_on_input``, :201),
    activation + requant, GEMM2 (routed weight otherwise, :217, top_k = 1),
    slot sum (:223-226).  ``hidden`` bf16-as-fp32 [M, H]; ``w1`` int8
    [E, 2I, H]; ``w2`` int8 [E, H, I].  Returns [M, H] (and a dict of every
    stage if ``stages``).
    """
    M, H = hidden.shape
    tw, ids = topk_softmax(logits, topk, renormalize)
    q_h, s_h = quant_per_token(hidden)
    c1 = grouped_gemm_w8a8(
        q_h, s_h, w1, s_w1, ids, topk, routed=tw if apply_router_weight_on_input else None
    )
    q_a, s_a, act = act_and_mul_quant(c1, activation)
    c3 = grouped_gemm_w8a8(
        q_a, s_a, w2, s_w2, ids, 1, routed=None if apply_router_weight_on_input else tw
    )
    out = moe_sum_reduce(c3.reshape(M, topk, H))
    if stages:
        return out, dict(
            topk_weights=tw, topk_ids=ids, q_h=q_h, s_h=s_h, cache1=c1, act=act,
            q_a=q_a, s_a=s_a, cache3=c3,
        )
    return out


# --------------------------------------------------------------------------
# Fused RMSNorm (+ residual) and per-token requant: the next step upstream
# of the path.  Replaces flashinfer rmsnorm / fused_add_rmsnorm
# (python/minisgl/layers/norm.py:8-38; called at
# python/minisgl/models/qwen3.py:37-40) followed by the quantizer of the
# W8A8 linear that consumes the normalised activations.
# --------------------------------------------------------------------------
def rmsnorm_quant(
    x: np.ndarray,
    weight: np.ndarray,
    eps: float,
    residual: Optional[np.ndarray] = None,
):
    """Closed form (every value a float32 array holding bf16 values):

    ``h = x`` or ``h = bf16(x + residual)`` (fp32 add, RNE narrowing; the
    new residual), ``ss = sum_k h_k^2`` exactly, ``ms = fp32(ss / H)``,
    ``r = 1 / sqrt(ms + eps)`` in fp32 IEEE arithmetic,
    ``y = bf16((h * r) * w)`` with each product rounded to fp32, then
    ``(q, s) = quant_per_token(y)``.

    ``ss`` is summed in float64 here: each square of a bf16 value is exact
    in float64, and the sum of at most 32768 of them is exact unless the
    squares span more than ~2^38 in magnitude, far outside activations.

    Returns (q int8 [M, H], s fp32 [M], y fp32 [M, H], h fp32 [M, H]).
    """
    x = np.asarray(x, _F32)
    M, H = x.shape
    w = np.asarray(weight, _F32).reshape(1, H)
    h = x if residual is None else bf16_round((x + np.asarray(residual, _F32)).astype(_F32))
    ss = (h.astype(np.float64) ** 2).sum(axis=1)
    ms = (ss / np.float64(H)).astype(_F32)
    r = (_F32(1.0) / np.sqrt(ms + _F32(eps), dtype=_F32)).astype(_F32)
    y = bf16_round(((h * r[:, None]).astype(_F32) * w).astype(_F32))
    q, s_ = quant_per_token(y)
    return q, s_, y, h
