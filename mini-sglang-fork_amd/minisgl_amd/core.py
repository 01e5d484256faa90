"""The slice of the reference's global Context that the MoE slot reads:
``ctx.moe_backend`` (python/minisgl/core.py:100-136, looked up at
python/minisgl/layers/moe.py:46-47).  Request/batch state is out of scope."""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional


@dataclass
class Context:
    moe_backend: Optional[object] = None


_GLOBAL_CTX: Optional[Context] = None


def set_global_ctx(ctx: Context) -> None:
    global _GLOBAL_CTX
    _GLOBAL_CTX = ctx


def get_global_ctx() -> Context:
    if _GLOBAL_CTX is None:
        raise RuntimeError("global context not set: call set_global_ctx(Context(moe_backend=...))")
    return _GLOBAL_CTX


def reset_global_ctx() -> None:
    global _GLOBAL_CTX
    _GLOBAL_CTX = None
