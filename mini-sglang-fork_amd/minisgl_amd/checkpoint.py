"""W8A8 checkpoint format and loader: the on-disk side of the path.

Format (safetensors, the reference's per-projection key names):

* every linear projection ``<p>.{q,k,v,o,gate,up,down}_proj`` stores
  ``<...>.weight`` int8 [N, K] (the reference's [out, in] layout) and
  ``<...>.weight_scale`` fp32 [N] (``weight = rint(w / weight_scale)``,
  ``weight_scale = amax_k |w| / 127`` per output channel); a bias stays bf16;
* the MoE router ``<p>.mlp.gate`` stays bf16, as the reference's router is a
  bf16 ``LinearReplicated`` (python/minisgl/models/utils.py:62-66): top-k
  selection is discontinuous, so int8 router logits could send a token to
  other experts than the bf16 router does;
* expert projections ``<p>.experts.<i>.{gate,up,down}_proj`` likewise;
* everything else (embeddings, norms, lm_head) stays bf16.

``load_w8a8`` mirrors the reference's streaming loader
(python/minisgl/models/weight.py:76-124): tensor-parallel sharding, merging
q|k|v and gate|up along dim 0, and stacking experts into [E, ...] tensors --
with three changes the int8 format needs:

* dtypes are preserved (the engine casts every loaded tensor to the model
  dtype, python/minisgl/engine/engine.py:146; int8 weights and fp32 scales
  must not be cast);
* row-parallel layers (o_proj, down_proj) split ``weight`` along dim 1 but
  replicate ``weight_scale`` [N] and the bias (the reference's
  ``chunk(dim=1)`` at python/minisgl/models/weight.py:43-44 would fail on a
  1-D tensor);
* stacked expert scales are renamed to the MoE layer's attribute names
  ``gate_up_scale`` / ``down_scale`` (a dotted packed name such as
  ``gate_up_proj.weight_scale`` cannot be a ``BaseOP`` attribute,
  python/minisgl/layers/base.py:22-26).

``quantize_checkpoint`` turns a bf16 state dict into the format on the GPU
(the same per-row HIP quantizer as the activations); ``dummy_w8a8_state``
replaces the engine's ``randn_like`` dummy weights
(python/minisgl/engine/engine.py:141-144), which are invalid for int8.
"""

from __future__ import annotations

import glob
import os
import re
from typing import Dict, Iterator, Optional, Tuple

import torch

_SPLIT_DIM_0 = (".q_proj", ".k_proj", ".v_proj", ".gate_proj", ".up_proj")
_SPLIT_DIM_1 = (".o_proj", ".down_proj")
_MERGE_GROUPS = {
    ".q_proj": (".qkv_proj", ("q", "k", "v")),
    ".k_proj": (".qkv_proj", ("q", "k", "v")),
    ".v_proj": (".qkv_proj", ("q", "k", "v")),
    ".gate_proj": (".gate_up_proj", ("gate", "up")),
    ".up_proj": (".gate_up_proj", ("gate", "up")),
}
_SLOT = {".q_proj": "q", ".k_proj": "k", ".v_proj": "v", ".gate_proj": "gate", ".up_proj": "up"}
_EXPERT = re.compile(r"^(?P<prefix>.+\.experts)\.(?P<idx>\d+)\.(?P<name>.+)$")
# packed expert tensor names -> MoE layer attributes
_EXPERT_RENAME = {
    "gate_up_proj.weight": "gate_up_proj",
    "down_proj.weight": "down_proj",
    "gate_up_proj.weight_scale": "gate_up_scale",
    "down_proj.weight_scale": "down_scale",
}
_QUANTIZED = re.compile(r"_proj\.weight$")


def is_quantized_weight(key: str) -> bool:
    """True for the keys stored as int8 + weight_scale."""
    return _QUANTIZED.search(key) is not None and "embed_tokens" not in key and "lm_head" not in key


def _shard(key: str, t: torch.Tensor, rank: int, size: int, num_kv_heads: Optional[int]) -> torch.Tensor:
    if size == 1:
        return t
    if any(s in key for s in _SPLIT_DIM_0):
        if any(s in key for s in (".k_proj", ".v_proj")) and num_kv_heads is not None and num_kv_heads < size:
            head_dim = t.shape[0] // num_kv_heads
            head = rank * num_kv_heads // size
            return t[head * head_dim : (head + 1) * head_dim].clone()
        return t.chunk(size, dim=0)[rank].clone()
    if any(s in key for s in _SPLIT_DIM_1):
        if t.dim() == 1:  # weight_scale [N] and bias [N] of a row-parallel layer
            return t
        return t.chunk(size, dim=1)[rank].clone()
    if "lm_head" in key or "embed_tokens" in key:
        per = -(-t.shape[0] // size)
        return t[rank * per : min((rank + 1) * per, t.shape[0])].clone()
    return t


def _merge_info(key: str):
    for suffix, (fused, slots) in _MERGE_GROUPS.items():
        if suffix in key:
            return key.replace(suffix, fused), _SLOT[suffix], slots
    return None


def _expert_info(key: str):
    m = _EXPERT.match(key)
    if m is None:
        return None
    name = m.group("name")
    name = _EXPERT_RENAME.get(name, name.removesuffix(".weight"))
    return f"{m.group('prefix')}.{name}", int(m.group("idx"))


def _files(path: str) -> list:
    if os.path.isfile(path):
        return [path]
    files = sorted(glob.glob(os.path.join(path, "*.safetensors")))
    return [f for f in files if not f.endswith("consolidated.safetensors")] or files


def load_w8a8(
    path: str,
    device: torch.device | str = "cpu",
    *,
    tp_rank: int = 0,
    tp_size: int = 1,
    num_kv_heads: Optional[int] = None,
    num_experts: Optional[int] = None,
    dtype: torch.dtype = torch.bfloat16,
) -> Iterator[Tuple[str, torch.Tensor]]:
    """Stream (name, tensor) pairs of a W8A8 checkpoint, sharded for
    ``tp_rank`` of ``tp_size``, merged and expert-stacked, on ``device``:
    int8 weights and fp32 scales keep their dtype, other tensors become
    ``dtype``."""
    import safetensors

    merge_buf: Dict[str, Dict[str, torch.Tensor]] = {}
    expert_buf: Dict[str, Dict[int, torch.Tensor]] = {}
    for file in _files(path):
        with safetensors.safe_open(file, framework="pt", device=str(device)) as f:
            for name in f.keys():
                if name.startswith(("vision_tower.", "multi_modal_projector.")):
                    continue
                raw = f.get_tensor(name)
                name = name.removeprefix("language_model.")
                t = _shard(name, raw, tp_rank, tp_size, num_kv_heads)
                if t.dtype not in (torch.int8, torch.float32):
                    t = t.to(dtype)
                elif t.dtype == torch.float32 and not name.endswith(".weight_scale"):
                    t = t.to(dtype)
                info = _merge_info(name)
                if info is None:
                    out = (name, t)
                else:
                    merged, slot, slots = info
                    merge_buf.setdefault(merged, {})[slot] = t
                    if not all(s in merge_buf[merged] for s in slots):
                        continue
                    group = merge_buf.pop(merged)
                    out = (merged, torch.cat([group[s] for s in slots], dim=0))
                einfo = _expert_info(out[0]) if num_experts else None
                if einfo is not None:
                    packed, idx = einfo
                    slots_e = expert_buf.setdefault(packed, {})
                    slots_e[idx] = out[1]
                    if len(slots_e) != num_experts:
                        continue
                    del expert_buf[packed]
                    yield packed, torch.stack([slots_e[i] for i in range(num_experts)], dim=0)
                else:
                    yield out
    if merge_buf:
        raise RuntimeError(f"incomplete merge groups in checkpoint: {sorted(merge_buf)}")
    if expert_buf:
        raise RuntimeError(f"incomplete expert tensors in checkpoint: {sorted(expert_buf)}")


def load_w8a8_state_dict(path: str, device: torch.device | str = "cpu", **kw) -> Dict[str, torch.Tensor]:
    """The whole checkpoint as a state dict for ``BaseOP.load_state_dict``
    (the engine's ``_load_weight_state_dict`` without the dtype cast)."""
    return dict(load_w8a8(path, device, **kw))


def quantize_checkpoint(state: Dict[str, torch.Tensor]) -> Dict[str, torch.Tensor]:
    """bf16 checkpoint -> W8A8 format: each quantized key's [N, K] weight
    becomes int8 ``weight`` + fp32 ``weight_scale`` (one HIP quantizer call
    per tensor, on the tensor's GPU); other tensors pass through."""
    from .kernel import quant_per_token

    out: Dict[str, torch.Tensor] = {}
    for key, t in state.items():
        if is_quantized_weight(key):
            if not t.is_cuda:
                raise ValueError(f"{key}: quantize_checkpoint needs GPU tensors (no CPU fallback)")
            if t.dim() != 2:
                raise ValueError(f"{key}: expected a [N, K] projection weight, got {tuple(t.shape)}")
            q, s = quant_per_token(t.to(torch.bfloat16).contiguous())
            out[key] = q
            out[key.removesuffix(".weight") + ".weight_scale"] = s
        else:
            out[key] = t
    return out


def save_w8a8(state: Dict[str, torch.Tensor], path: str) -> None:
    """Write a W8A8 state dict (from ``quantize_checkpoint``) as safetensors."""
    from safetensors.torch import save_file

    save_file({k: v.detach().contiguous().cpu() for k, v in state.items()}, path)


def dummy_w8a8_state(
    template: Dict[str, torch.Tensor], device: torch.device | str, seed: int = 0
) -> Dict[str, torch.Tensor]:
    """Random weights for a W8A8 model's state dict (the engine's
    ``--dummy-weight`` path): int8 uniform in [-127, 127], fp32 scales in
    [1e-3, 1e-2], other tensors ``randn`` in their own dtype."""
    gen = torch.Generator(device=device).manual_seed(seed)
    out: Dict[str, torch.Tensor] = {}
    for key, v in template.items():
        if v.dtype == torch.int8:
            out[key] = torch.randint(-127, 128, tuple(v.shape), generator=gen, dtype=torch.int8, device=device)
        elif v.dtype == torch.float32:
            out[key] = torch.rand(tuple(v.shape), generator=gen, device=device) * 9e-3 + 1e-3
        else:
            out[key] = torch.randn(tuple(v.shape), generator=gen, device=device).to(v.dtype)
    return out


__all__ = [
    "is_quantized_weight",
    "load_w8a8",
    "load_w8a8_state_dict",
    "quantize_checkpoint",
    "save_w8a8",
    "dummy_w8a8_state",
]
