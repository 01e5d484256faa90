from .registry import Registry


def div_even(a: int, b: int, allow_replicate: bool = False) -> int:
    """``a / b`` that must divide evenly (python/minisgl/utils misc helper);
    with ``allow_replicate`` a smaller ``a`` is replicated (returns 1 share)."""
    if allow_replicate and a < b:
        assert b % a == 0, f"{b} is not a multiple of {a}"
        return 1
    assert a % b == 0, f"{a} is not divisible by {b}"
    return a // b


def div_ceil(a: int, b: int) -> int:
    return -(-a // b)


__all__ = ["Registry", "div_even", "div_ceil"]
