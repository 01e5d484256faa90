"""ctypes binding of libmw8.so (the C ABI declared in include/mw8.h).

The library is built in-tree by ``__graft_entry__.build()`` (hipcc,
--offload-arch=gfx950) and sits next to this file.  There is no fallback:
if the library is missing every op raises.

The reference binds its native kernels through tvm-ffi modules
(python/minisgl/kernel/utils.py:53-129); this module plays that role for a
plain C ABI.
"""

from __future__ import annotations

import ctypes
import functools
import os
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p

LIB_NAME = "libmw8.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)
# the benchmark's measurement kernels (include/mw8_calib.h), a library of their own
CALIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libmw8_calib.so")

_P = c_void_p
_I32 = c_int32
_I64 = c_int64

# name -> (restype, argtypes); must match include/mw8.h
SIGNATURES = {
    "mw8_last_error": (ctypes.c_char_p, []),
    "mw8_version": (ctypes.c_int, []),
    "mw8_device_info": (ctypes.c_int, [_I32, _P, _P, _P]),
    "mw8_quant_per_token_bf16": (ctypes.c_int, [_P, _I64, _I64, _I64, _P, _I64, _P, _P]),
    "mw8_act_and_mul_quant_bf16": (ctypes.c_int, [_P, _I64, _I64, _I32, _P, _P, _P, _P]),
    "mw8_set_tuning": (None, [_I32, _I32, _I32]),
    "mw8_gemm_workspace_bytes": (c_size_t, [_I64, _I64, _I64]),
    "mw8_gemm_workspace_max_bytes": (c_size_t, []),
    "mw8_tuning_count": (_I32, [_I32]),
    "mw8_gemm_kernel_name": (ctypes.c_char_p, [_I64, _I64, _I64]),
    "mw8_gemm_w8a8_bf16": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P, c_size_t, _P],
    ),
    "mw8_gemm_w8a8_bf16_noalloc": (ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "mw8_gemm_w8a8_i32": (ctypes.c_int, [_P, _P, _P, _I64, _I64, _I64, _P, c_size_t, _P]),
    "mw8_gemm_act_w8a8_bf16": (ctypes.c_int, [_P, _P, _P, _P, _I32, _P, _I64, _I64, _I64, _P, c_size_t, _P]),
    "mw8_gemm_act_supported": (_I32, [_I64, _I64, _I64]),
    "mw8_gemm_act_workspace_bytes": (c_size_t, [_I64, _I64, _I64]),
    "mw8_linear_bf16_w8a8": (ctypes.c_int, [_P, _I64, _P, _P, _P, _P, _I64, _I64, _I64, _P]),
    "mw8_linear_bf16_supported": (_I32, [_I64, _I64, _I64]),
    "mw8_topk_softmax": (ctypes.c_int, [_P, _I32, _I64, _I32, _I32, _I32, _P, _P, _P]),
    "mw8_moe_align_max_padded": (_I64, [_I64, _I32, _I32]),
    "mw8_moe_align_block_size": (ctypes.c_int, [_P, _I64, _I32, _I32, _P, _P, _P, _P]),
    "mw8_moe_gemm_w8a8_bf16": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _I32, _I64, _I64, _I64, _I32, _I32, _P, _P],
    ),
    "mw8_moe_gemm_w8a8_i32": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _I64, _I32, _I64, _I64, _I64, _I32, _I32, _P, _P],
    ),
    "mw8_moe_sum_reduce_bf16": (ctypes.c_int, [_P, _I64, _I32, _I64, _P, _P]),
    "mw8_moe_gemm_act_w8a8_bf16": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _I32, _I64, _I64, _I64, _I32, _I32, _I32, _P, _P],
    ),
    "mw8_moe_gemm_sum_w8a8_bf16": (
        ctypes.c_int,
        [_P, _P, _P, _P, _P, _P, _P, _I64, _P, _I32, _I64, _I64, _I64, _I32, _P, _P],
    ),
    "mw8_moe_gemm_sum_supported": (_I32, [_I64, _I64, _I32]),
    "mw8_moe_gemm_topk_w8a8_bf16": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I32, _P, _P]
    ),
    "mw8_moe_gemm_sum_topk_w8a8_bf16": (
        ctypes.c_int, [_P, _P, _P, _P, _P, _P, _I32, _I64, _I64, _I64, _I32, _P, _P]
    ),
    "mw8_moe_route_quant": (
        ctypes.c_int, [_P, _I32, _I64, _I32, _I32, _I32, _P, _I64, _P, _P, _P, _P, _P]
    ),
    "mw8_moe_prepare_small": (
        ctypes.c_int,
        [_P, _I32, _I64, _I32, _I32, _I32, _P, _I64, _P, _P, _P, _P, _I32, _I32, _P, _P, _P, _P],
    ),
    "mw8_rmsnorm_quant_bf16": (ctypes.c_int, [_P, _P, _P, c_float, _I64, _I64, _P, _P, _P, _P]),
    "mw8_rmsnorm_strided_bf16": (ctypes.c_int, [_P, _I64, _P, _I64, _P, c_float, _I64, _I64, _I64, _P]),
}

ERROR_NAMES = {
    1: "MW8_ERR_ARG",
    2: "MW8_ERR_SHAPE",
    3: "MW8_ERR_ALIGN",
    4: "MW8_ERR_WORKSPACE",
    5: "MW8_ERR_LAUNCH",
}


class MW8Error(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"{ERROR_NAMES.get(code, code)}: {message}")
        self.code = code


@functools.lru_cache(maxsize=None)
def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load libmw8.so and declare every entry point; raises if it is missing."""
    if not os.path.exists(path):
        raise RuntimeError(
            f"{path} not found: build the HIP library first (python -c "
            "'import __graft_entry__ as g; g.build()')"
        )
    lib = ctypes.CDLL(path)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def check(rc: int) -> None:
    if rc != 0:
        msg = load().mw8_last_error().decode(errors="replace")
        raise MW8Error(rc, msg)


# name -> (restype, argtypes); must match include/mw8_calib.h
CALIB_SIGNATURES = {
    "mw8_calib_last_error": (ctypes.c_char_p, []),
    "mw8_calib_sink_len": (_I64, []),
    "mw8_calib_mfma_i8": (ctypes.c_int, [_I32, _I32, _P, _I64, _P]),
    "mw8_calib_read": (ctypes.c_int, [_P, _I64, _P, _I64, _P]),
    "mw8_calib_stream_lds": (ctypes.c_int, [_P, _I64, _I32, _I32, _P, _I64, _P]),
}


@functools.lru_cache(maxsize=None)
def load_calib(path: str = CALIB_PATH) -> ctypes.CDLL:
    """Load libmw8_calib.so (benchmark measurement kernels only)."""
    if not os.path.exists(path):
        raise RuntimeError(f"{path} not found: build the HIP libraries first")
    lib = ctypes.CDLL(path)
    for name, (res, args) in CALIB_SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


def check_calib(rc: int) -> None:
    if rc != 0:
        raise MW8Error(rc, load_calib().mw8_calib_last_error().decode(errors="replace"))


__all__ = ["load", "check", "load_calib", "check_calib", "MW8Error", "LIB_PATH", "CALIB_PATH", "SIGNATURES",
           "CALIB_SIGNATURES", "c_float"]
