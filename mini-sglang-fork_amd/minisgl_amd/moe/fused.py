"""W8A8 fused-MoE backend: the orchestration of fused_experts_impl
(python/minisgl/moe/fused.py:127-227) over HIP kernels.

Flow for M tokens, top-k slots, E experts, w1 int8 [E, N=2I, H],
w2 int8 [E, H, I]:

1. route: ``topk_softmax`` (fp32 softmax, top-k, double renormalisation)
2. ``moe_align_block_size`` with BLOCK_SIZE_M from ``get_default_config``
3. quantize ``hidden_states`` once per token (GEMM1 addresses A rows as
   ``pair // top_k``)
4. GEMM1 -> bf16 cache [M*k, N]; routed weight only if
   ``apply_router_weight_on_input`` (reference :201)
5. activation + requant -> int8 [M*k, I] + fp32 scales (prefill batches:
   the activation runs in GEMM1's epilogue, then the plain quantizer)
6. GEMM2 (top_k = 1) -> bf16 cache [M*k, H], routed weight otherwise (:217)
7. slot sum, written into ``hidden_states`` in place (:175, :223-226);
   decode batches (16-row blocks) run 6 and 7 as one kernel
   (``fused_moe_kernel_sum_w8a8``), the same bits without the cache

All counts stay on the device (no host sync), so the call can be captured
in a HIP graph.  For the smallest decode batches (M * k <= 32) the backend
runs steps 1-3 as one launch (``moe_prepare_small``), otherwise steps 1 and
3 as one launch (``moe_route_quant``), with the same outputs bit for bit.

Any hidden size H and intermediate size I: the int8 kernels contract over
multiples of 16 bytes, so a layer whose H or I is not one runs on copies
zero-padded to the next multiple of 16 (``padded_experts_w8a8``): hidden
columns past H, gate and up rows past I and down columns past I are zero.
Zero terms leave every int32 sum as it is, a zero gate and up row gives
``act(0) * 0 = 0`` (silu and gelu), which leaves each row's amax, scale and
quantized values as they are, and the result is the unpadded problem's bit
for bit (the reference's Triton kernel masks its K tail instead,
python/minisgl/kernel/triton/fused_moe.py:159-174).
"""

from __future__ import annotations

import functools
from typing import Dict, Tuple

import torch

from ..kernel import (
    act_and_mul_quant,
    fused_moe_kernel_act_w8a8,
    fused_moe_kernel_sum_topk_w8a8,
    fused_moe_kernel_sum_w8a8,
    fused_moe_kernel_topk_w8a8,
    fused_moe_kernel_w8a8,
    moe_align_block_size,
    moe_gemm_sum_supported,
    moe_prepare_small,
    moe_route_quant,
    moe_sum_reduce,
    quant_per_token,
    topk_softmax,
    TOPK_ROWS_KERNEL_MAX_TOKENS,
)
from .base import BaseMoeBackend

# Tokens up to which decode batches skip the alignment pass: the grouped
# GEMMs take each expert's pairs straight from the router ids (the router
# picks distinct experts per token, so an expert holds at most one pair per
# token, at most 16 here).  Measured on MI355X at config 3 (layer, us,
# router-id rows vs the best aligned path): 1 token 27.5 vs 29.6, 2 tokens
# 32.7 vs 35.0, 4 tokens 44.2 vs 49.1, 5 tokens 49.8 vs 52.5, 8 tokens 58.6
# vs 62.6, 16 tokens 84.8 vs 87.2.  The kernels take up to 48 tokens (two or
# three 16-pair units per expert), but there every block's scan of the
# router ids costs more than the alignment launch: 17 / 32 / 48 tokens 90.6
# / 111.3 / 131.6 vs 88.6 / 107.3 / 112.3.
TOPK_ROWS_MAX_TOKENS = 16
assert TOPK_ROWS_MAX_TOKENS <= TOPK_ROWS_KERNEL_MAX_TOKENS, "the dispatch limit stays within the kernels' limit"

# Pairs (tokens x top-k) up to which the backend runs router, alignment and
# hidden quantization as one launch, where the router-id rows do not apply
# (more than 256 experts).  The kernel accepts up to 1024 pairs, but one
# block serialises what the separate kernels spread over the GPU: measured
# on MI355X at config 3 (layer, us, one launch vs three): 1 token 30.4 vs
# 32.0, 4 tokens 52.5 vs 54.0, 8 tokens 70.0 vs 70.1, 16 tokens 97.9 vs
# 96.4, 64 tokens 159.1 vs 133.7.
PREPARE_MAX_PAIRS = 32


def fused_topk(
    hidden_states: torch.Tensor,
    gating_output: torch.Tensor,
    topk: int,
    renormalize: bool,
    num_token_non_padded: torch.Tensor | None = None,
) -> Tuple[torch.Tensor, torch.Tensor]:
    """(topk_weights fp32 [M, k], topk_ids int32 [M, k]); one HIP kernel
    (python/minisgl/moe/fused.py:9-28).  Tokens at or past
    ``num_token_non_padded`` (a device tensor, so no host sync) get ids -1,
    which the alignment skips (:25-27)."""
    assert hidden_states.shape[0] == gating_output.shape[0], "Number of tokens mismatch"
    topk_weights, topk_ids = topk_softmax(gating_output.contiguous(), topk, renormalize)
    if num_token_non_padded is not None:
        indices = torch.arange(0, topk_ids.shape[0], device=topk_ids.device)
        topk_ids[indices >= num_token_non_padded, :] = -1
    return topk_weights, topk_ids


def get_default_config(M: int, E: int, N: int, K: int, topk: int) -> Dict[str, int]:
    """Two tile regimes keyed on tokens vs experts, as the reference
    (python/minisgl/moe/fused.py:92-113), with the same keys.  BLOCK_SIZE_M
    is the alignment block: 16 rows when M <= E (decode: weight streaming),
    otherwise 64 (MFMA tiles).  The other keys describe this build's
    kernels for that regime: the weight rows a block streams and the K
    bytes of one ring stage (16 rows x 256 bytes for 16-row blocks; 128 or
    256 columns x 64 bytes for the tile walk), and GROUP_SIZE_M = 1 (the
    tiles are ordered per XCD instead of by a GROUP_M swizzle)."""
    if M <= E:
        return {"BLOCK_SIZE_M": 16, "BLOCK_SIZE_N": 16, "BLOCK_SIZE_K": 256, "GROUP_SIZE_M": 1}
    return {"BLOCK_SIZE_M": 64, "BLOCK_SIZE_N": 128, "BLOCK_SIZE_K": 64, "GROUP_SIZE_M": 1}


def try_get_optimal_moe_config(w1_shape, w2_shape, top_k: int, M: int) -> Dict[str, int]:
    E, _, N = w2_shape
    return get_default_config(M, E, N, w1_shape[2], top_k)


def _up16(n: int) -> int:
    return -(-n // 16) * 16


def padded_experts_w8a8(w1, w1_scale, w2, w2_scale):
    """(w1, w1_scale, w2, w2_scale) with H and I zero-padded to multiples of
    16: w1 [E, 2 I16, H16] with gate rows at [0, I) and up rows at
    [I16, I16 + I), w1_scale [E, 2 I16], w2 [E, H16, I16], w2_scale
    [E, H16]; padded rows get a zero scale.  The copies are cached on ``w1``
    and rebuilt when any of the four tensors is replaced or written in place
    (data pointer and version counter), so a captured graph replays on the
    copies its warm-up call made."""
    E, N, H = w1.shape
    I = N // 2
    H16, I16 = _up16(H), _up16(I)
    key = (H16, I16) + tuple((t.data_ptr(), t._version, tuple(t.shape)) for t in (w1, w1_scale, w2, w2_scale))
    hit = getattr(w1, "_mw8_padded", None)
    if hit is not None and hit[0] == key:
        return hit[1]
    w1p = w1.new_zeros((E, 2, I16, H16))
    w1p[:, :, :I, :H] = w1.view(E, 2, I, H)
    s1p = w1_scale.new_zeros((E, 2, I16))
    s1p[:, :, :I] = w1_scale.reshape(E, 2, I)
    w2p = w2.new_zeros((E, H16, I16))
    w2p[:, :H, :I] = w2
    s2p = w2_scale.new_zeros((E, H16))
    s2p[:, :H] = w2_scale.reshape(E, H)
    out = (w1p.view(E, 2 * I16, H16), s1p.view(E, 2 * I16), w2p, s2p)
    w1._mw8_padded = (key, out)
    return out


def _padded_hidden(hidden_states: torch.Tensor) -> torch.Tensor:
    M, H = hidden_states.shape
    hp = hidden_states.new_zeros((M, _up16(H)))
    hp[:, :H] = hidden_states
    return hp


def fused_experts_impl_w8a8(
    hidden_states: torch.Tensor,
    w1: torch.Tensor,
    w1_scale: torch.Tensor,
    w2: torch.Tensor,
    w2_scale: torch.Tensor,
    topk_weights: torch.Tensor,
    topk_ids: torch.Tensor,
    activation: str = "silu",
    apply_router_weight_on_input: bool = False,
) -> torch.Tensor:
    assert hidden_states.shape[1] == w1.shape[2], "Hidden size mismatch"
    assert topk_weights.shape == topk_ids.shape, "topk shape mismatch"
    assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
    assert w1.is_contiguous(), "Expert weights1 must be contiguous"
    assert w2.is_contiguous(), "Expert weights2 must be contiguous"
    assert hidden_states.dtype == torch.bfloat16, "W8A8 MoE takes bf16 activations"
    assert w1.dtype == torch.int8 and w2.dtype == torch.int8, "W8A8 MoE takes int8 weights"
    M, H = hidden_states.shape
    E, N, _ = w1.shape
    k = topk_ids.shape[1]
    if H % 16 != 0 or (N // 2) % 16 != 0:
        hp = _padded_hidden(hidden_states)
        w1p, s1p, w2p, s2p = padded_experts_w8a8(w1, w1_scale, w2, w2_scale)
        fused_experts_impl_w8a8(
            hp, w1p, s1p, w2p, s2p, topk_weights, topk_ids, activation, apply_router_weight_on_input
        )
        return hidden_states.copy_(hp[:, :H])
    config = functools.partial(try_get_optimal_moe_config, w1.shape, w2.shape, k)(M)
    bsz = config["BLOCK_SIZE_M"]

    sorted_ids, expert_ids, num_post_pad = moe_align_block_size(topk_ids, bsz, E)
    q_h, s_h = quant_per_token(hidden_states)
    return _experts_from_routing(
        hidden_states, q_h, s_h, w1, w1_scale, w2, w2_scale, topk_weights, sorted_ids, expert_ids,
        num_post_pad, k, bsz, activation, apply_router_weight_on_input,
    )


def _experts_from_routing(
    hidden_states, q_h, s_h, w1, w1_scale, w2, w2_scale, topk_weights, sorted_ids, expert_ids,
    num_post_pad, k, bsz, activation, apply_router_weight_on_input,
) -> torch.Tensor:
    """Steps 4-7: GEMM1, activation + requant, GEMM2, slot sum in place.
    Prefill batches (>= 32 pairs per expert, 64/128-row blocks) run the
    activation in GEMM1's epilogue, writing [M*k, I] instead of [M*k, 2I];
    decode batches (16-row blocks) run the slot sum inside GEMM2, which
    writes hidden_states directly; the values are the same bit for bit."""
    M, H = hidden_states.shape
    E, N, K = w1.shape
    if bsz == 16 and moe_gemm_sum_supported(sorted_ids.shape[0], M * k, E):
        cache1 = torch.empty((M * k, N), dtype=torch.bfloat16, device=hidden_states.device)
        fused_moe_kernel_w8a8(
            q_h, s_h, w1, w1_scale, cache1, topk_weights, sorted_ids, expert_ids, num_post_pad,
            apply_router_weight_on_input, k, bsz, M * k,
        )
        q_a, s_a = act_and_mul_quant(cache1, activation)
        fused_moe_kernel_sum_w8a8(
            q_a, s_a, w2, w2_scale, hidden_states, None if apply_router_weight_on_input else topk_weights,
            sorted_ids, expert_ids, num_post_pad, k, M * k,
        )
        return hidden_states
    # one buffer backs both bf16 caches, as in the reference (:157-172)
    cache = torch.empty(M * k * max(N, H), dtype=torch.bfloat16, device=hidden_states.device)
    if bsz in (64, 128) and M * k >= 32 * E and N % 16 == 0 and K % 64 == 0 and E < 512:
        act = cache[: M * k * (N // 2)].view(M * k, N // 2)
        fused_moe_kernel_act_w8a8(
            q_h, s_h, w1, w1_scale, act, sorted_ids, expert_ids, num_post_pad, k, bsz, M * k,
            activation, topk_weights if apply_router_weight_on_input else None,
        )
        q_a, s_a = quant_per_token(act)
    else:
        cache1 = cache[: M * k * N].view(M * k, N)
        fused_moe_kernel_w8a8(
            q_h, s_h, w1, w1_scale, cache1, topk_weights, sorted_ids, expert_ids, num_post_pad,
            apply_router_weight_on_input, k, bsz, M * k,
        )
        q_a, s_a = act_and_mul_quant(cache1, activation)
    cache3 = cache[: M * k * H].view(M * k, H)
    fused_moe_kernel_w8a8(
        q_a, s_a, w2, w2_scale, cache3, topk_weights, sorted_ids, expert_ids, num_post_pad,
        not apply_router_weight_on_input, 1, bsz, M * k,
    )
    moe_sum_reduce(cache3.view(M, k, H), hidden_states)
    return hidden_states


def _experts_from_router_ids(
    hidden_states, q_h, s_h, w1, w1_scale, w2, w2_scale, topk_weights, topk_ids, activation,
    apply_router_weight_on_input,
) -> torch.Tensor:
    """Steps 4-7 for a decode batch without the alignment: GEMM1 over each
    expert's pairs listed from topk_ids, activation + requant, GEMM2 with
    the slot sum writing hidden_states; bit-identical to
    _experts_from_routing with 16-row blocks."""
    M, _ = hidden_states.shape
    _, N, _ = w1.shape
    k = topk_ids.shape[1]
    cache1 = torch.empty((M * k, N), dtype=torch.bfloat16, device=hidden_states.device)
    fused_moe_kernel_topk_w8a8(
        q_h, s_h, w1, w1_scale, cache1, topk_ids, topk_weights if apply_router_weight_on_input else None
    )
    q_a, s_a = act_and_mul_quant(cache1, activation)
    fused_moe_kernel_sum_topk_w8a8(
        q_a, s_a, w2, w2_scale, hidden_states, topk_ids, None if apply_router_weight_on_input else topk_weights
    )
    return hidden_states


class FusedMoeW8A8(BaseMoeBackend):
    def forward(
        self,
        hidden_states: torch.Tensor,
        w1: torch.Tensor,
        w2: torch.Tensor,
        gating_output: torch.Tensor,
        topk: int,
        renormalize: bool,
        activation: str = "silu",
        apply_router_weight_on_input: bool = False,
        w1_scale: torch.Tensor | None = None,
        w2_scale: torch.Tensor | None = None,
        **kwargs,
    ) -> torch.Tensor:
        if w1_scale is None or w2_scale is None:
            raise ValueError("the W8A8 MoE backend needs w1_scale and w2_scale")
        M, H = hidden_states.shape
        E = w1.shape[0]
        if w1.shape[1] != 2 * w2.shape[2] or w2.shape[1] != H:
            raise ValueError(
                f"W8A8 MoE takes w1 [E, 2I, H] and w2 [E, H, I] "
                f"(got w1 {tuple(w1.shape)}, w2 {tuple(w2.shape)}, hidden size {H})"
            )
        # the contract fused_experts_impl_w8a8 asserts, for the fast paths too
        assert H == w1.shape[2], "Hidden size mismatch"
        assert hidden_states.dtype == torch.bfloat16, "W8A8 MoE takes bf16 activations"
        assert w1.dtype == torch.int8 and w2.dtype == torch.int8, "W8A8 MoE takes int8 weights"
        assert w1.is_contiguous() and w2.is_contiguous(), "Expert weights must be contiguous"
        if H % 16 != 0 or w2.shape[2] % 16 != 0:
            # the int8 kernels contract over multiples of 16: run on zero-padded
            # copies (same bits), then write the H real columns back in place
            assert hidden_states.is_contiguous(), "Hidden_states must be contiguous"
            hp = _padded_hidden(hidden_states)
            w1p, s1p, w2p, s2p = padded_experts_w8a8(w1, w1_scale, w2, w2_scale)
            self.forward(
                hp, w1p, w2p, gating_output, topk, renormalize, activation, apply_router_weight_on_input,
                w1_scale=s1p, w2_scale=s2p,
            )
            return hidden_states.copy_(hp[:, :H])
        bsz = try_get_optimal_moe_config(w1.shape, w2.shape, topk, M)["BLOCK_SIZE_M"]
        contiguous = hidden_states.is_contiguous() and gating_output.is_contiguous()
        if (
            contiguous
            and bsz == 16
            and 0 < M <= TOPK_ROWS_MAX_TOKENS
            and E <= 256
            and moe_gemm_sum_supported(16 * E * -(-M // 16), M * topk, E)
        ):
            # decode batch: router + hidden quantization in one launch, then
            # the grouped GEMMs list each expert's pairs from the router ids
            # (no alignment launch)
            topk_weights, topk_ids, q_h, s_h = moe_route_quant(gating_output, hidden_states, topk, renormalize)
            return _experts_from_router_ids(
                hidden_states, q_h, s_h, w1, w1_scale, w2, w2_scale, topk_weights, topk_ids, activation,
                apply_router_weight_on_input,
            )
        if (
            bsz == 16
            and 0 < M * topk <= PREPARE_MAX_PAIRS
            and E + 1 <= 512
            and hidden_states.is_contiguous()
            and gating_output.is_contiguous()
        ):
            # decode batch: router, alignment and hidden quantization in one launch
            topk_weights, _, sorted_ids, expert_ids, npp, q_h, s_h = moe_prepare_small(
                gating_output, hidden_states, topk, renormalize, bsz, E
            )
            return _experts_from_routing(
                hidden_states, q_h, s_h, w1, w1_scale, w2, w2_scale, topk_weights, sorted_ids,
                expert_ids, npp, topk, bsz, activation, apply_router_weight_on_input,
            )
        if hidden_states.is_contiguous() and gating_output.is_contiguous():
            # router and hidden quantization in one launch (one wave per token)
            topk_weights, topk_ids, q_h, s_h = moe_route_quant(gating_output, hidden_states, topk, renormalize)
            sorted_ids, expert_ids, npp = moe_align_block_size(topk_ids, bsz, E)
            return _experts_from_routing(
                hidden_states, q_h, s_h, w1, w1_scale, w2, w2_scale, topk_weights, sorted_ids, expert_ids,
                npp, topk, bsz, activation, apply_router_weight_on_input,
            )
        # step by step (a non-contiguous router output, or a non-contiguous
        # hidden_states, which fused_experts_impl_w8a8 rejects as the
        # reference does, python/minisgl/moe/fused.py:140-145)
        topk_weights, topk_ids = fused_topk(hidden_states, gating_output, topk, renormalize)
        return fused_experts_impl_w8a8(
            hidden_states, w1, w1_scale, w2, w2_scale, topk_weights, topk_ids, activation,
            apply_router_weight_on_input=apply_router_weight_on_input,
        )


__all__ = [
    "fused_topk",
    "get_default_config",
    "try_get_optimal_moe_config",
    "fused_experts_impl_w8a8",
    "padded_experts_w8a8",
    "FusedMoeW8A8",
]
