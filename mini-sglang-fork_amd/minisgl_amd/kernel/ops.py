"""torch-facing wrappers over the HIP C ABI.

Every function validates shapes/dtypes on the host, allocates outputs with
torch (the caching allocator, so the calls stay capturable in a HIP graph),
and launches on the current torch stream.  Nothing here computes on the
CPU: a missing library or a non-GPU tensor raises.
"""

from __future__ import annotations

from typing import Dict, Optional, Tuple

import torch

from .lib import check, load

_ACT = {"silu": 0, "gelu": 1}


def _stream(t: torch.Tensor) -> int:
    return torch.cuda.current_stream(t.device).cuda_stream


def _ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _need(cond: bool, msg: str) -> None:
    if not cond:
        raise ValueError(msg)


def _on_gpu(*ts: Optional[torch.Tensor]) -> None:
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("the W8A8 HIP path needs GPU tensors (no CPU fallback)")


def _same_device(*ts: Optional[torch.Tensor]) -> None:
    devs = {t.device for t in ts if t is not None}
    if len(devs) > 1:
        raise ValueError(f"the W8A8 HIP path needs every tensor on one device, got {sorted(map(str, devs))}")


# ----------------------------------------------------------------- workspace
_WORKSPACE: Dict[torch.device, torch.Tensor] = {}


def reserve_gemm_workspace(device: torch.device) -> torch.Tensor:
    """A reserved GEMM workspace for ``device``, for callers that drive the
    C entry points themselves (``gemm_w8a8`` and ``gemm_w8a8_i32`` take a
    per-call workspace from torch's caching allocator instead): one buffer of
    ``mw8_gemm_workspace_max_bytes()`` (the bound over every shape and
    tiling, 64 MiB on a 256-CU MI355X), allocated on first use and never
    grown, replaced or freed.  So a HIP graph that captured a GEMM keeps a
    valid workspace pointer whatever runs later, and no call inside a
    capture allocates once the workspace exists (the reference engine runs
    each batch size eagerly before capturing it, which reserves it,
    python/minisgl/engine/graph.py:129-144).  The buffer holds int32
    partial tiles only during one call, so calls ordered on one stream
    share it; calls on concurrent streams must not."""
    dev = torch.device(device)
    if dev.index is None:
        dev = torch.device(dev.type, torch.cuda.current_device())
    ws = _WORKSPACE.get(dev)
    if ws is None:
        with torch.cuda.device(dev):
            need = int(load().mw8_gemm_workspace_max_bytes())
        ws = torch.empty(max(need, 16), dtype=torch.uint8, device=dev)
        _WORKSPACE[dev] = ws
    return ws


def _call_workspace(M: int, N: int, K: int, device: torch.device) -> Optional[torch.Tensor]:
    """The K split's int32 partial tiles for one call at (M, N, K), or None
    when no split applies: a buffer from torch's caching allocator, which
    hands a freed block back only to work ordered after its last use on the
    same stream (and takes it from the graph's private pool under capture),
    so calls on concurrent streams never share one.  The size is planned for
    q's device and the calling thread's tuning override, as the call is."""
    with torch.cuda.device(device):
        need = int(load().mw8_gemm_workspace_bytes(M, N, K))
    return torch.empty(need, dtype=torch.uint8, device=device) if need > 0 else None


def gemm_workspace(M: int, N: int, K: int, device: torch.device) -> Optional[torch.Tensor]:
    """Workspace for the GEMM's K split at (M, N, K): the device's reserved
    buffer (reserve_gemm_workspace), or None when no split applies."""
    if int(load().mw8_gemm_workspace_bytes(M, N, K)) == 0:
        return None
    return reserve_gemm_workspace(device)


# ----------------------------------------------------------------- quantizer
def quant_per_token(
    x: torch.Tensor, out: Optional[torch.Tensor] = None, scale: Optional[torch.Tensor] = None
) -> Tuple[torch.Tensor, torch.Tensor]:
    """bf16 [M, K] -> (int8 [M, K], fp32 [M]); s = amax/127, q = rint(x/s)."""
    _on_gpu(x)
    _need(x.dtype == torch.bfloat16 and x.dim() == 2, "quant_per_token: x must be bf16 [M, K]")
    _need(x.stride(1) == 1, "quant_per_token: last dim must be contiguous")
    M, K = x.shape
    q = out if out is not None else torch.empty((M, K), dtype=torch.int8, device=x.device)
    s = scale if scale is not None else torch.empty((M,), dtype=torch.float32, device=x.device)
    _need(q.dtype == torch.int8 and q.shape == (M, K) and q.stride(1) == 1, "bad q buffer")
    _need(s.dtype == torch.float32 and s.shape == (M,) and s.is_contiguous(), "bad s buffer")
    if M == 0:
        return q, s
    check(
        load().mw8_quant_per_token_bf16(
            _ptr(x), M, K, x.stride(0), _ptr(q), q.stride(0), _ptr(s), _stream(x)
        )
    )
    return q, s


def act_and_mul_quant(
    x: torch.Tensor, activation: str = "silu", return_act: bool = False, quantize: bool = True,
    act_out: Optional[torch.Tensor] = None,
):
    """bf16 [R, 2d] -> (int8 [R, d], fp32 [R][, bf16 act [R, d]]);
    ``quantize=False`` computes the activation only and returns it."""
    _on_gpu(x, act_out)
    _need(activation in _ACT, f"unsupported activation {activation}")
    _need(x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(), "x: bf16 [R, 2d]")
    R, two_d = x.shape
    d = two_d // 2
    q = torch.empty((R, d), dtype=torch.int8, device=x.device) if quantize else None
    s = torch.empty((R,), dtype=torch.float32, device=x.device) if quantize else None
    a = act_out
    if a is None and (return_act or not quantize):
        a = torch.empty((R, d), dtype=torch.bfloat16, device=x.device)
    if a is not None:
        _need(a.dtype == torch.bfloat16 and a.shape == (R, d) and a.is_contiguous(), "act_out: bf16 [R, d]")
    if R > 0:
        check(
            load().mw8_act_and_mul_quant_bf16(
                _ptr(x), R, two_d, _ACT[activation], _ptr(q), _ptr(s), _ptr(a), _stream(x)
            )
        )
    if not quantize:
        return a
    return (q, s, a) if return_act else (q, s)


def rmsnorm_quant(
    x: torch.Tensor,
    weight: torch.Tensor,
    eps: float,
    residual: Optional[torch.Tensor] = None,
    y: Optional[torch.Tensor] = None,
    return_y: bool = False,
    quantize: bool = True,
):
    """Fused RMSNorm (+ residual add, in place) and per-token int8 quant.

    bf16 x [M, H] -> (int8 q [M, H], fp32 s [M][, bf16 y [M, H]]).  With
    ``residual`` the norm runs on ``bf16(x + residual)``, which is written
    back into ``residual`` (the reference's fused_add_rmsnorm contract,
    python/minisgl/layers/norm.py:33-38).  ``y`` may be ``x`` itself.
    ``quantize=False`` skips the quantizer and returns ``y`` only.
    """
    _on_gpu(x, weight, residual, y)
    _need(x.dtype == torch.bfloat16 and x.dim() == 2 and x.is_contiguous(), "x: bf16 [M, H] contiguous")
    M, H = x.shape
    _need(weight.dtype == torch.bfloat16 and weight.shape == (H,) and weight.is_contiguous(), "weight: bf16 [H]")
    if residual is not None:
        _need(residual.dtype == torch.bfloat16 and residual.shape == (M, H) and residual.is_contiguous(),
              "residual: bf16 [M, H] contiguous")
    if (return_y or not quantize) and y is None:
        y = torch.empty((M, H), dtype=torch.bfloat16, device=x.device)
    if y is not None:
        _need(y.dtype == torch.bfloat16 and y.shape == (M, H) and y.is_contiguous(), "y: bf16 [M, H]")
    q = torch.empty((M, H), dtype=torch.int8, device=x.device) if quantize else None
    s = torch.empty((M,), dtype=torch.float32, device=x.device) if quantize else None
    if M > 0:
        check(
            load().mw8_rmsnorm_quant_bf16(
                _ptr(x), _ptr(residual), _ptr(weight), float(eps), M, H, _ptr(q), _ptr(s), _ptr(y),
                _stream(x),
            )
        )
    if not quantize:
        return y
    return (q, s, y) if (return_y or y is not None) else (q, s)


def _row_groups(t: torch.Tensor) -> Optional[Tuple[int, int, int]]:
    """(G, inner, ld) if the rows of ``t`` [..., H] sit at g * ld + i * H
    (g < G, i < inner, the last dim contiguous), else None."""
    if t.dim() < 2 or t.stride(-1) != 1:
        return None
    H = t.shape[-1]
    if t.is_contiguous():
        return t.numel() // H, 1, H
    if t.dim() == 2:
        G, inner, ld = t.shape[0], 1, (t.stride(0) if t.shape[0] > 1 else H)
    elif t.dim() == 3 and (t.stride(1) == H or t.shape[1] == 1):
        G, inner, ld = t.shape[0], t.shape[1], (t.stride(0) if t.shape[0] > 1 else t.shape[1] * H)
    else:
        return None
    return (G, inner, ld) if ld >= inner * H else None


def rmsnorm_strided(x: torch.Tensor, weight: torch.Tensor, eps: float, out: Optional[torch.Tensor] = None) -> bool:
    """Plain RMSNorm of the rows of a strided view ``x`` [G, inner, H] (or
    [R, H] with a row stride) into ``out`` (default: in place, ``out = x``).
    Returns False when the layout is not expressible as [G, inner, H] row
    groups with 16-byte aligned rows (the caller then copies)."""
    out = x if out is None else out
    _on_gpu(x, weight, out)
    _need(x.dtype == torch.bfloat16 and out.dtype == torch.bfloat16 and x.shape == out.shape, "x/out: bf16, same shape")
    H = x.shape[-1]
    _need(weight.dtype == torch.bfloat16 and weight.shape == (H,) and weight.is_contiguous(), "weight: bf16 [H]")
    gx, go = _row_groups(x), _row_groups(out)
    if gx is not None and out.is_contiguous():
        # a contiguous out holds x's row groups back to back: g * (inner * H) + i * H
        go = (gx[0], gx[1], gx[1] * H)
    if gx is None or go is None or gx[:2] != go[:2] or H % 8 or gx[2] % 8 or go[2] % 8:
        return False
    if x.data_ptr() % 16 or out.data_ptr() % 16:
        return False
    G, inner, ldx = gx
    if G * inner > 0:
        check(
            load().mw8_rmsnorm_strided_bf16(
                _ptr(x), ldx, _ptr(out), go[2], _ptr(weight), float(eps), G, inner, H, _stream(x)
            )
        )
    return True


# ----------------------------------------------------------------- dense GEMM
def _check_gemm(q: torch.Tensor, w: torch.Tensor) -> Tuple[int, int, int]:
    _on_gpu(q, w)
    _need(q.dtype == torch.int8 and q.dim() == 2 and q.is_contiguous(), "A: int8 [M, K] contiguous")
    _need(w.dtype == torch.int8 and w.dim() == 2 and w.is_contiguous(), "W: int8 [N, K] contiguous")
    _need(q.shape[1] == w.shape[1], "A/W K mismatch")
    return q.shape[0], w.shape[0], q.shape[1]


def gemm_w8a8(
    q: torch.Tensor,
    s_a: torch.Tensor,
    w: torch.Tensor,
    s_w: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """y bf16 [M, N] = bf16(((acc * s_a[m]) * s_w[n]) + bias[n])."""
    M, N, K = _check_gemm(q, w)
    _need(s_a.dtype == torch.float32 and s_a.shape == (M,) and s_a.is_contiguous(), "s_a: fp32 [M]")
    _need(s_w.dtype == torch.float32 and s_w.shape == (N,) and s_w.is_contiguous(), "s_w: fp32 [N]")
    if bias is not None:
        _need(bias.dtype == torch.bfloat16 and bias.shape == (N,) and bias.is_contiguous(), "bias: bf16 [N]")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=q.device)
    _need(y.dtype == torch.bfloat16 and y.shape == (M, N) and y.is_contiguous(), "bad out buffer")
    if M == 0:
        return y
    ws = _call_workspace(M, N, K, q.device)
    with torch.cuda.device(q.device):  # the library plans the tiling for the current device
        check(
            load().mw8_gemm_w8a8_bf16(
                _ptr(q), _ptr(s_a), _ptr(w), _ptr(s_w), _ptr(bias), _ptr(y), M, N, K, _ptr(ws),
                0 if ws is None else ws.numel(), _stream(q),
            )
        )
    return y


# Rows from which the gated MLP runs gate_up with the activation in its
# epilogue.  MI355X, us, two-step (GEMM into [M, 2I], activation + requant)
# -> fused (gemm_act_w8a8, then the requant of [M, I]): M 2080, I 25600
# 625-641 -> 587-597; M 2080, I 6400 157-161 -> 154; M 4096 / 8192, I 17408
# 693-703 -> 672, 1307-1311 -> 1262-1264; below it the two-step path is as
# fast or faster (M 512, I 17408 124 -> 127; M 256, I 768 13.4 -> 28).
GEMM_ACT_MIN_ROWS = 1024


def gemm_act_supported(M: int, I: int, K: int) -> bool:
    """Whether gemm_act_w8a8 takes (M, I, K) (host only; follows the tile
    override): I % 8 == 0, K % 128 == 0 and a shape the plain GEMM at
    (M, 2I, K) runs on its ring cores."""
    return bool(load().mw8_gemm_act_supported(M, I, K))


def gemm_act_w8a8(
    q: torch.Tensor,
    s_a: torch.Tensor,
    w: torch.Tensor,
    s_w: torch.Tensor,
    activation: str = "silu",
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """y bf16 [M, I] = bf16(act(g) * u) of the W8A8 GEMM against a gate|up
    weight w int8 [2I, K] (gate rows first; s_w fp32 [2I]): bit for bit
    act_and_mul_quant(gemm_w8a8(q, s_a, w, s_w), activation,
    return_act=True)[2], without the [M, 2I] gate|up output
    (gemm_act_supported shapes)."""
    M, N2, K = _check_gemm(q, w)
    _need(N2 % 2 == 0, "W: [2I, K] gate|up rows")
    I = N2 // 2
    _need(activation in _ACT, f"unsupported activation {activation}")
    _need(s_a.dtype == torch.float32 and s_a.shape == (M,) and s_a.is_contiguous(), "s_a: fp32 [M]")
    _need(s_w.dtype == torch.float32 and s_w.shape == (N2,) and s_w.is_contiguous(), "s_w: fp32 [2I]")
    y = out if out is not None else torch.empty((M, I), dtype=torch.bfloat16, device=q.device)
    _need(y.dtype == torch.bfloat16 and y.shape == (M, I) and y.is_contiguous(), "bad out buffer")
    if M == 0:
        return y
    with torch.cuda.device(q.device):
        need = int(load().mw8_gemm_act_workspace_bytes(M, I, K))
    ws = torch.empty(need, dtype=torch.uint8, device=q.device) if need > 0 else None
    with torch.cuda.device(q.device):
        check(
            load().mw8_gemm_act_w8a8_bf16(
                _ptr(q), _ptr(s_a), _ptr(w), _ptr(s_w), _ACT[activation], _ptr(y), M, I, K, _ptr(ws),
                0 if ws is None else ws.numel(), _stream(q),
            )
        )
    return y


def linear_bf16_supported(M: int, N: int, K: int) -> bool:
    """Whether linear_bf16_w8a8 takes a decode batch of this shape (host
    only; the answer follows the decode-configuration override)."""
    return bool(load().mw8_linear_bf16_supported(M, N, K))


def linear_bf16_w8a8(
    x: torch.Tensor,
    w: torch.Tensor,
    s_w: torch.Tensor,
    bias: Optional[torch.Tensor] = None,
    out: Optional[torch.Tensor] = None,
) -> torch.Tensor:
    """y bf16 [M, N] = the W8A8 linear of bf16 x [M, K] in one launch
    (per-token quantization inside the decode GEMM), bit for bit
    gemm_w8a8(*quant_per_token(x), w, s_w, bias).  Decode batches only
    (linear_bf16_supported); x rows 16-byte aligned, last dim contiguous."""
    _on_gpu(x, w, s_w, bias, out)
    _need(x.dtype == torch.bfloat16 and x.dim() == 2 and x.stride(1) == 1, "x: bf16 [M, K], rows contiguous")
    _need(w.dtype == torch.int8 and w.dim() == 2 and w.is_contiguous() and w.shape[1] == x.shape[1], "W: int8 [N, K]")
    M, K = x.shape
    N = w.shape[0]
    _need(s_w.dtype == torch.float32 and s_w.shape == (N,) and s_w.is_contiguous(), "s_w: fp32 [N]")
    if bias is not None:
        _need(bias.dtype == torch.bfloat16 and bias.shape == (N,) and bias.is_contiguous(), "bias: bf16 [N]")
    y = out if out is not None else torch.empty((M, N), dtype=torch.bfloat16, device=x.device)
    _need(y.dtype == torch.bfloat16 and y.shape == (M, N) and y.is_contiguous(), "bad out buffer")
    ldx = x.stride(0) if M > 1 else K
    check(
        load().mw8_linear_bf16_w8a8(
            _ptr(x), ldx, _ptr(w), _ptr(s_w), _ptr(bias), _ptr(y), M, N, K, _stream(x),
        )
    )
    return y


def gemm_w8a8_i32(q: torch.Tensor, w: torch.Tensor) -> torch.Tensor:
    """Raw int32 accumulators acc [M, N] = A . W^T (parity hook)."""
    M, N, K = _check_gemm(q, w)
    acc = torch.empty((M, N), dtype=torch.int32, device=q.device)
    if M == 0:
        return acc
    ws = _call_workspace(M, N, K, q.device)
    with torch.cuda.device(q.device):
        check(
            load().mw8_gemm_w8a8_i32(
                _ptr(q), _ptr(w), _ptr(acc), M, N, K, _ptr(ws), 0 if ws is None else ws.numel(),
                _stream(q),
            )
        )
    return acc


# ----------------------------------------------------------------- MoE pieces
def topk_softmax(
    gating_output: torch.Tensor, topk: int, renormalize: bool
) -> Tuple[torch.Tensor, torch.Tensor]:
    """Router: fp32 softmax, top-k, optional double renormalisation.

    Mirrors fused_topk (python/minisgl/moe/fused.py:9-28), including the
    extra ``w / (sum(w) + 1e-8)`` of :23-24, in one kernel.
    """
    _on_gpu(gating_output)
    g = gating_output
    _need(g.dim() == 2 and g.is_contiguous(), "gating_output: [M, E] contiguous")
    _need(g.dtype in (torch.bfloat16, torch.float32), "gating_output: bf16 or fp32")
    M, E = g.shape
    w = torch.empty((M, topk), dtype=torch.float32, device=g.device)
    ids = torch.empty((M, topk), dtype=torch.int32, device=g.device)
    if M > 0:
        check(
            load().mw8_topk_softmax(
                _ptr(g), int(g.dtype == torch.bfloat16), M, E, topk, int(renormalize),
                _ptr(w), _ptr(ids), _stream(g),
            )
        )
    return w, ids


def moe_align_block_size(
    topk_ids: torch.Tensor, block_size: int, num_experts: int
) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Same contract and buffer sizes as python/minisgl/moe/fused.py:31-89
    (``num_experts + 1`` expert slots, sentinel ``numel`` padding).  Pairs
    inside one expert segment are in ascending flat order."""
    _on_gpu(topk_ids)
    _need(topk_ids.dtype == torch.int32 and topk_ids.is_contiguous(), "topk_ids: int32 contiguous")
    lib = load()
    numel = topk_ids.numel()
    slots = num_experts + 1
    max_padded = int(lib.mw8_moe_align_max_padded(numel, slots, block_size))
    max_blocks = -(-max_padded // block_size)
    dev = topk_ids.device
    sorted_ids = torch.empty((max_padded,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((max_blocks,), dtype=torch.int32, device=dev)
    num_tokens_post_pad = torch.empty((1,), dtype=torch.int32, device=dev)
    check(
        lib.mw8_moe_align_block_size(
            _ptr(topk_ids), numel, slots, block_size, _ptr(sorted_ids), _ptr(expert_ids),
            _ptr(num_tokens_post_pad), _stream(topk_ids),
        )
    )
    return sorted_ids, expert_ids, num_tokens_post_pad


PREPARE_MAX_PAIRS = 1024  # M * topk bound of the one-block preparation


def moe_route_quant(
    gating_output: torch.Tensor,
    hidden_states: torch.Tensor,
    topk: int,
    renormalize: bool,
) -> Tuple[torch.Tensor, ...]:
    """Router + hidden-state quantization in one launch (one wave per
    token).  Returns (topk_weights fp32 [M, k], topk_ids int32 [M, k], q
    int8 [M, H], s fp32 [M]), bit-identical to topk_softmax and
    quant_per_token."""
    _on_gpu(gating_output, hidden_states)
    g, h = gating_output, hidden_states
    _need(g.dim() == 2 and g.is_contiguous(), "gating_output: [M, E] contiguous")
    _need(g.dtype in (torch.bfloat16, torch.float32), "gating_output: bf16 or fp32")
    _need(h.dtype == torch.bfloat16 and h.dim() == 2 and h.is_contiguous(), "hidden_states: bf16 [M, H] contiguous")
    M, E = g.shape
    _need(h.shape[0] == M, "hidden_states / gating_output token counts differ")
    H = h.shape[1]
    dev = g.device
    w = torch.empty((M, topk), dtype=torch.float32, device=dev)
    ids = torch.empty((M, topk), dtype=torch.int32, device=dev)
    q = torch.empty((M, H), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    check(
        load().mw8_moe_route_quant(
            _ptr(g), int(g.dtype == torch.bfloat16), M, E, topk, int(renormalize), _ptr(h), H,
            _ptr(w), _ptr(ids), _ptr(q), _ptr(s), _stream(g),
        )
    )
    return w, ids, q, s


def moe_prepare_small(
    gating_output: torch.Tensor,
    hidden_states: torch.Tensor,
    topk: int,
    renormalize: bool,
    block_size: int,
    num_experts: int,
) -> Tuple[torch.Tensor, ...]:
    """Router + alignment + hidden-state quantization in one launch (decode
    batches, M * topk <= 1024).  Returns (topk_weights, topk_ids, sorted_ids,
    expert_ids, num_tokens_post_pad, q, s), each bit-identical to
    topk_softmax, moe_align_block_size and quant_per_token."""
    _on_gpu(gating_output, hidden_states)
    g, h = gating_output, hidden_states
    _need(g.dim() == 2 and g.is_contiguous(), "gating_output: [M, E] contiguous")
    _need(g.dtype in (torch.bfloat16, torch.float32), "gating_output: bf16 or fp32")
    _need(h.dtype == torch.bfloat16 and h.dim() == 2 and h.is_contiguous(), "hidden_states: bf16 [M, H] contiguous")
    M, E = g.shape
    _need(h.shape[0] == M, "hidden_states / gating_output token counts differ")
    _need(E == num_experts, "gating_output width != num_experts")
    H = h.shape[1]
    lib = load()
    dev = g.device
    slots = num_experts + 1
    numel = M * topk
    max_padded = int(lib.mw8_moe_align_max_padded(numel, slots, block_size))
    max_blocks = -(-max_padded // block_size)
    w = torch.empty((M, topk), dtype=torch.float32, device=dev)
    ids = torch.empty((M, topk), dtype=torch.int32, device=dev)
    q = torch.empty((M, H), dtype=torch.int8, device=dev)
    s = torch.empty((M,), dtype=torch.float32, device=dev)
    sorted_ids = torch.empty((max_padded,), dtype=torch.int32, device=dev)
    expert_ids = torch.empty((max_blocks,), dtype=torch.int32, device=dev)
    npp = torch.empty((1,), dtype=torch.int32, device=dev)
    check(
        lib.mw8_moe_prepare_small(
            _ptr(g), int(g.dtype == torch.bfloat16), M, E, topk, int(renormalize), _ptr(h), H,
            _ptr(w), _ptr(ids), _ptr(q), _ptr(s), slots, block_size, _ptr(sorted_ids),
            _ptr(expert_ids), _ptr(npp), _stream(g),
        )
    )
    return w, ids, sorted_ids, expert_ids, npp, q, s


def fused_moe_kernel_w8a8(
    A: torch.Tensor,
    A_scale: torch.Tensor,
    B: torch.Tensor,
    B_scale: torch.Tensor,
    C: torch.Tensor,
    topk_weights: torch.Tensor,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    mul_routed_weight: bool,
    top_k: int,
    block_size: int,
    num_valid_tokens: int,
) -> None:
    """Grouped W8A8 GEMM, the counterpart of fused_moe_kernel_triton
    (python/minisgl/kernel/moe_impl.py:6-62): row p of C (a flat
    (token, slot) pair, C viewed as [M*k, N]) receives
    ``epilogue(A[p // top_k] . B[e]^T)``, times ``topk_weights[p]`` if
    ``mul_routed_weight``."""
    _on_gpu(A, A_scale, B, B_scale, C)
    _need(A.dtype == torch.int8 and A.dim() == 2 and A.is_contiguous(), "A: int8 [T, K]")
    _need(B.dtype == torch.int8 and B.dim() == 3 and B.is_contiguous(), "B: int8 [E, N, K]")
    E, N, K = B.shape
    _need(A.shape[1] == K, "A/B K mismatch")
    _need(A_scale.dtype == torch.float32 and A_scale.shape == (A.shape[0],), "A_scale: fp32 [T]")
    _need(B_scale.dtype == torch.float32 and B_scale.shape == (E, N) and B_scale.is_contiguous(), "B_scale: fp32 [E, N]")
    _need(C.dtype == torch.bfloat16 and C.is_contiguous() and C.numel() == num_valid_tokens * N, "C: bf16 [M*k, N]")
    assert topk_weights.stride(1) == 1  # python/minisgl/kernel/moe_impl.py:25
    assert sorted_token_ids.stride(0) == 1  # :26
    check(
        load().mw8_moe_gemm_w8a8_bf16(
            _ptr(A), _ptr(A_scale), _ptr(B), _ptr(B_scale), _ptr(sorted_token_ids),
            _ptr(expert_ids), _ptr(num_tokens_post_padded), sorted_token_ids.shape[0],
            _ptr(topk_weights) if mul_routed_weight else None, top_k, num_valid_tokens, N, K, E,
            block_size, _ptr(C), _stream(A),
        )
    )


def fused_moe_kernel_act_w8a8(
    A: torch.Tensor,
    A_scale: torch.Tensor,
    B: torch.Tensor,
    B_scale: torch.Tensor,
    C: torch.Tensor,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    top_k: int,
    block_size: int,
    num_valid_tokens: int,
    activation: str = "silu",
    topk_weights: Optional[torch.Tensor] = None,
) -> None:
    """Gate|up grouped GEMM with the gated activation in its epilogue
    (``topk_weights`` given: the routed weight multiplies g and u first):
    C bf16 [M*k, N/2] = act(gate) * up, bit-identical to
    fused_moe_kernel_w8a8 into [M*k, N] followed by act_and_mul_quant's
    activation (64/128-row blocks, persistent walk)."""
    _on_gpu(A, A_scale, B, B_scale, C)
    _need(A.dtype == torch.int8 and A.dim() == 2 and A.is_contiguous(), "A: int8 [T, K]")
    _need(B.dtype == torch.int8 and B.dim() == 3 and B.is_contiguous(), "B: int8 [E, N, K]")
    E, N, K = B.shape
    _need(A.shape[1] == K, "A/B K mismatch")
    _need(A_scale.dtype == torch.float32 and A_scale.shape == (A.shape[0],), "A_scale: fp32 [T]")
    _need(B_scale.dtype == torch.float32 and B_scale.shape == (E, N) and B_scale.is_contiguous(), "B_scale: fp32 [E, N]")
    _need(C.dtype == torch.bfloat16 and C.is_contiguous() and C.numel() == num_valid_tokens * (N // 2), "C: bf16 [M*k, N/2]")
    _need(activation in ("silu", "gelu"), "activation: silu or gelu")
    check(
        load().mw8_moe_gemm_act_w8a8_bf16(
            _ptr(A), _ptr(A_scale), _ptr(B), _ptr(B_scale), _ptr(sorted_token_ids), _ptr(expert_ids),
            _ptr(num_tokens_post_padded), sorted_token_ids.shape[0], _ptr(topk_weights), top_k,
            num_valid_tokens, N, K, E, block_size, 0 if activation == "silu" else 1, _ptr(C), _stream(A),
        )
    )


def fused_moe_kernel_w8a8_i32(
    A: torch.Tensor,
    B: torch.Tensor,
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    top_k: int,
    block_size: int,
    num_valid_tokens: int,
) -> torch.Tensor:
    """Raw int32 accumulators of the grouped GEMM, [num_valid, N] (parity hook)."""
    _on_gpu(A, B)
    E, N, K = B.shape
    out = torch.zeros((num_valid_tokens, N), dtype=torch.int32, device=A.device)
    check(
        load().mw8_moe_gemm_w8a8_i32(
            _ptr(A), _ptr(B), _ptr(sorted_token_ids), _ptr(expert_ids),
            _ptr(num_tokens_post_padded), sorted_token_ids.shape[0], top_k, num_valid_tokens,
            N, K, E, block_size, _ptr(out), _stream(A),
        )
    )
    return out


def moe_gemm_sum_supported(max_sorted: int, num_valid: int, num_experts: int) -> bool:
    """Whether fused_moe_kernel_sum_w8a8 takes these routing sizes (its LDS
    tables fit one block); host only."""
    return bool(load().mw8_moe_gemm_sum_supported(max_sorted, num_valid, num_experts))


def fused_moe_kernel_sum_w8a8(
    A: torch.Tensor,
    A_scale: torch.Tensor,
    B: torch.Tensor,
    B_scale: torch.Tensor,
    output: torch.Tensor,
    topk_weights: Optional[torch.Tensor],
    sorted_token_ids: torch.Tensor,
    expert_ids: torch.Tensor,
    num_tokens_post_padded: torch.Tensor,
    top_k: int,
    num_valid_tokens: int,
) -> None:
    """Down-projection grouped GEMM with the top-k slot sum fused in, for
    16-row alignment blocks: output bf16 [M, N] receives, bit for bit, what
    fused_moe_kernel_w8a8 (pair rows, routed weight from ``topk_weights``
    unless None) followed by moe_sum_reduce writes (python/minisgl/moe/fused.py:212-226)."""
    _on_gpu(A, A_scale, B, B_scale, output, topk_weights, sorted_token_ids, expert_ids, num_tokens_post_padded)
    _same_device(A, A_scale, B, B_scale, output, topk_weights, sorted_token_ids, expert_ids, num_tokens_post_padded)
    _need(A.dtype == torch.int8 and A.dim() == 2 and A.is_contiguous(), "A: int8 [M*k, K]")
    _need(B.dtype == torch.int8 and B.dim() == 3 and B.is_contiguous(), "B: int8 [E, N, K]")
    E, N, K = B.shape
    _need(A.shape == (num_valid_tokens, K), "A: int8 [M*k, K]")
    _need(A_scale.dtype == torch.float32 and A_scale.shape == (num_valid_tokens,), "A_scale: fp32 [M*k]")
    _need(B_scale.dtype == torch.float32 and B_scale.shape == (E, N) and B_scale.is_contiguous(), "B_scale: fp32 [E, N]")
    _need(num_valid_tokens % top_k == 0, "num_valid_tokens: a multiple of top_k")
    _need(output.dtype == torch.bfloat16 and output.is_contiguous() and output.shape == (num_valid_tokens // top_k, N),
          "output: bf16 [M, N]")
    _need(topk_weights is None or (topk_weights.dtype == torch.float32 and topk_weights.is_contiguous()
                                   and topk_weights.numel() == num_valid_tokens), "topk_weights: fp32 [M, k]")
    _need(sorted_token_ids.dtype == torch.int32 and sorted_token_ids.stride(0) == 1, "sorted_token_ids: int32")
    check(
        load().mw8_moe_gemm_sum_w8a8_bf16(
            _ptr(A), _ptr(A_scale), _ptr(B), _ptr(B_scale), _ptr(sorted_token_ids), _ptr(expert_ids),
            _ptr(num_tokens_post_padded), sorted_token_ids.shape[0], _ptr(topk_weights), top_k,
            num_valid_tokens, N, K, E, _ptr(output), _stream(A),
        )
    )


TOPK_ROWS_KERNEL_MAX_TOKENS = 48  # batches the router-id grouped GEMM kernels accept


def _check_topk_rows(A, A_scale, B, B_scale, topk_ids, topk_weights, pairs_per_row):
    _on_gpu(A, A_scale, B, B_scale, topk_ids, topk_weights)
    _same_device(A, A_scale, B, B_scale, topk_ids, topk_weights)
    _need(B.dtype == torch.int8 and B.dim() == 3 and B.is_contiguous(), "B: int8 [E, N, K]")
    E, N, K = B.shape
    _need(topk_ids.dtype == torch.int32 and topk_ids.dim() == 2 and topk_ids.is_contiguous(),
          "topk_ids: int32 [M, k] contiguous")
    M, k = topk_ids.shape
    _need(M <= TOPK_ROWS_KERNEL_MAX_TOKENS, f"router-id rows: at most {TOPK_ROWS_KERNEL_MAX_TOKENS} tokens")
    _need(A.dtype == torch.int8 and A.is_contiguous() and A.shape == (M * k if pairs_per_row else M, K),
          "A: int8 [M, K] (GEMM1) or [M*k, K] (GEMM2)")
    _need(A_scale.dtype == torch.float32 and A_scale.shape == (A.shape[0],), "A_scale: fp32 [rows of A]")
    _need(B_scale.dtype == torch.float32 and B_scale.shape == (E, N) and B_scale.is_contiguous(), "B_scale: fp32 [E, N]")
    _need(topk_weights is None or (topk_weights.dtype == torch.float32 and topk_weights.is_contiguous()
                                   and topk_weights.numel() == M * k), "topk_weights: fp32 [M, k]")
    return E, N, K, M, k


def fused_moe_kernel_topk_w8a8(
    A: torch.Tensor,
    A_scale: torch.Tensor,
    B: torch.Tensor,
    B_scale: torch.Tensor,
    C: torch.Tensor,
    topk_ids: torch.Tensor,
    topk_weights: Optional[torch.Tensor],
) -> None:
    """GEMM1 of a decode batch (at most 48 tokens, distinct experts per
    token) with each expert's rows taken from the router ids: C bf16
    [M*k, N] pair rows, bit-identical to moe_align_block_size(16) +
    fused_moe_kernel_w8a8 (python/minisgl/moe/fused.py:71-89, :192-205)."""
    E, N, K, M, k = _check_topk_rows(A, A_scale, B, B_scale, topk_ids, topk_weights, False)
    _need(C.dtype == torch.bfloat16 and C.is_contiguous() and C.shape == (M * k, N), "C: bf16 [M*k, N]")
    check(
        load().mw8_moe_gemm_topk_w8a8_bf16(
            _ptr(A), _ptr(A_scale), _ptr(B), _ptr(B_scale), _ptr(topk_ids), _ptr(topk_weights), k, M * k,
            N, K, E, _ptr(C), _stream(A),
        )
    )


def fused_moe_kernel_sum_topk_w8a8(
    A: torch.Tensor,
    A_scale: torch.Tensor,
    B: torch.Tensor,
    B_scale: torch.Tensor,
    output: torch.Tensor,
    topk_ids: torch.Tensor,
    topk_weights: Optional[torch.Tensor],
) -> None:
    """GEMM2 + top-k slot sum of a decode batch with the expert rows taken
    from the router ids: output bf16 [M, N], bit-identical to
    fused_moe_kernel_sum_w8a8 over a 16-row alignment."""
    E, N, K, M, k = _check_topk_rows(A, A_scale, B, B_scale, topk_ids, topk_weights, True)
    _need(output.dtype == torch.bfloat16 and output.is_contiguous() and output.shape == (M, N), "output: bf16 [M, N]")
    check(
        load().mw8_moe_gemm_sum_topk_w8a8_bf16(
            _ptr(A), _ptr(A_scale), _ptr(B), _ptr(B_scale), _ptr(topk_ids), _ptr(topk_weights), k, M * k,
            N, K, E, _ptr(output), _stream(A),
        )
    )


def moe_sum_reduce(input: torch.Tensor, output: torch.Tensor) -> None:
    """out[t] = bf16(sum_i in[t, i]) (python/minisgl/kernel/moe_impl.py:65-98)."""
    _on_gpu(input, output)
    assert input.is_contiguous() and output.is_contiguous()
    token_num, topk_num, hidden_dim = input.shape
    assert output.shape[0] == token_num and output.shape[1] == hidden_dim
    _need(input.dtype == torch.bfloat16 and output.dtype == torch.bfloat16, "bf16 only")
    check(
        load().mw8_moe_sum_reduce_bf16(
            _ptr(input), token_num, topk_num, hidden_dim, _ptr(output), _stream(input)
        )
    )


__all__ = [
    "moe_gemm_sum_supported",
    "fused_moe_kernel_sum_w8a8",
    "fused_moe_kernel_topk_w8a8",
    "fused_moe_kernel_sum_topk_w8a8",
    "TOPK_ROWS_KERNEL_MAX_TOKENS",
    "gemm_workspace",
    "reserve_gemm_workspace",
    "quant_per_token",
    "act_and_mul_quant",
    "rmsnorm_quant",
    "rmsnorm_strided",
    "gemm_w8a8",
    "gemm_w8a8_i32",
    "linear_bf16_supported",
    "GEMM_ACT_MIN_ROWS",
    "gemm_act_supported",
    "gemm_act_w8a8",
    "linear_bf16_w8a8",
    "topk_softmax",
    "moe_align_block_size",
    "fused_moe_kernel_w8a8",
    "fused_moe_kernel_w8a8_i32",
    "fused_moe_kernel_act_w8a8",
    "moe_prepare_small",
    "moe_route_quant",
    "moe_sum_reduce",
]
