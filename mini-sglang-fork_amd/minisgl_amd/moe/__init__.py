"""MoE backend registry (python/minisgl/moe/__init__.py:16-27).  The W8A8
backend registers under ``"fused_w8a8"``; the reference selects backends by
``--moe-backend`` (python/minisgl/server/args.py:213-218)."""

from __future__ import annotations

from typing import Protocol

from ..utils import Registry
from .base import BaseMoeBackend


class MoeBackendCreator(Protocol):
    def __call__(self) -> BaseMoeBackend: ...


SUPPORTED_MOE_BACKENDS = Registry[MoeBackendCreator]("MoE Backend")


@SUPPORTED_MOE_BACKENDS.register("fused_w8a8")
def create_fused_w8a8_moe_backend():
    from .fused import FusedMoeW8A8

    return FusedMoeW8A8()


def create_moe_backend(backend: str) -> BaseMoeBackend:
    return SUPPORTED_MOE_BACKENDS[backend]()


__all__ = ["BaseMoeBackend", "create_moe_backend", "SUPPORTED_MOE_BACKENDS"]
