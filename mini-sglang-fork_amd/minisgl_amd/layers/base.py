"""Parameter discovery and state-dict plumbing with the semantics of the
reference's BaseOP (python/minisgl/layers/base.py:15-99): every public
tensor attribute is a parameter, public BaseOP attributes recurse with a
dotted prefix, ``load_state_dict`` pops each key, requires equal shape and
dtype, rebinds the attribute, and rejects leftover keys at the top level."""

from __future__ import annotations

from typing import Any, Dict, Generic, List, TypeVar

import torch

StateDict = Dict[str, torch.Tensor]


def _join(prefix: str, name: str) -> str:
    return f"{prefix}.{name}" if prefix else name


class BaseOP:
    def forward(self, *args: Any, **kwargs: Any) -> Any:  # pragma: no cover - abstract
        raise NotImplementedError

    def _public_items(self):
        return [(k, v) for k, v in self.__dict__.items() if not k.startswith("_")]

    def state_dict(self, *, prefix: str = "", result: StateDict | None = None) -> StateDict:
        out: StateDict = {} if result is None else result
        for name, value in self._public_items():
            if isinstance(value, torch.Tensor):
                out[_join(prefix, name)] = value
            elif isinstance(value, BaseOP):
                value.state_dict(prefix=_join(prefix, name), result=out)
        return out

    def load_state_dict(self, state_dict: StateDict, *, prefix: str = "", _internal: bool = False) -> None:
        for name, value in self._public_items():
            key = _join(prefix, name)
            if isinstance(value, torch.Tensor):
                item = state_dict.pop(key)
                assert isinstance(item, torch.Tensor)
                if item.shape != value.shape or item.dtype != value.dtype:
                    raise AssertionError(
                        f"{key}: expected {tuple(value.shape)} {value.dtype}, "
                        f"got {tuple(item.shape)} {item.dtype}"
                    )
                setattr(self, name, item)
            elif isinstance(value, BaseOP):
                value.load_state_dict(state_dict, prefix=key, _internal=True)
        if not _internal and state_dict:
            raise RuntimeError(f"Unexpected keys in state_dict: {list(state_dict)}")


class StateLessOP(BaseOP):
    def state_dict(self, *, prefix: str = "", result: StateDict | None = None) -> StateDict:
        return {} if result is None else result

    def load_state_dict(self, state_dict: StateDict, *, prefix: str = "", _internal: bool = False) -> None:
        if not _internal and state_dict:
            raise RuntimeError(f"Unexpected keys in state_dict: {list(state_dict)}")


T = TypeVar("T", bound=BaseOP)


class OPList(BaseOP, Generic[T]):
    def __init__(self, ops: List[T]):
        self.op_list = ops

    def state_dict(self, *, prefix: str = "", result: StateDict | None = None) -> StateDict:
        out: StateDict = {} if result is None else result
        for i, op in enumerate(self.op_list):
            op.state_dict(prefix=_join(prefix, str(i)), result=out)
        return out

    def load_state_dict(self, state_dict: StateDict, *, prefix: str = "", _internal: bool = False) -> None:
        for i, op in enumerate(self.op_list):
            op.load_state_dict(state_dict, prefix=_join(prefix, str(i)), _internal=True)
        if not _internal and state_dict:
            raise RuntimeError(f"Unexpected keys in state_dict: {list(state_dict)}")
