"""Name -> factory registry with the behaviour of the reference's Registry
(python/minisgl/utils/registry.py:6-38): duplicate names raise KeyError,
unknown names raise KeyError, ``assert_supported`` raises ArgumentTypeError."""

from __future__ import annotations

from typing import Callable, Dict, Generic, Iterable, List, TypeVar

T = TypeVar("T")


class Registry(Generic[T]):
    def __init__(self, type: str):
        self._items: Dict[str, T] = {}
        self._type = type

    def register(self, name: str) -> Callable[[T], T]:
        if name in self._items:
            raise KeyError(f"{self._type} '{name}' is already registered.")

        def decorator(item: T) -> T:
            self._items[name] = item
            return item

        return decorator

    def __getitem__(self, name: str) -> T:
        if name not in self._items:
            raise KeyError(f"Unsupported {self._type}: {name}")
        return self._items[name]

    def supported_names(self) -> List[str]:
        return list(self._items)

    def assert_supported(self, names: str | Iterable[str]) -> None:
        from argparse import ArgumentTypeError

        for name in [names] if isinstance(names, str) else names:
            if name not in self._items:
                raise ArgumentTypeError(
                    f"Unsupported {self._type}: {name}. Supported items: {self.supported_names()}"
                )
