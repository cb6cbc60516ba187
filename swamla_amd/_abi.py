"""ctypes boundary to libswamla_mi355x.so (declared in include/swamla_mi355x.h).

The library is built in-tree by ``swamla_amd.build.build_library()``; this
module only loads it.  Every entry point returns an int status that is turned
into ``RuntimeError(mla_last_error())`` here, mirroring how the reference
raises from ATen on bad shapes (models/mla.py:413).
"""
from __future__ import annotations

import ctypes
import os
from typing import Optional

import torch

LIB_NAME = "libswamla_mi355x.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

ABI_VERSION = 6
DTYPE_F32, DTYPE_BF16, DTYPE_FP8 = 0, 1, 2
ERR_NAMES = {
    -1: "INVALID_ARG",
    -2: "UNSUPPORTED",
    -3: "MISALIGNED",
    -4: "OUT_OF_RANGE",
    -5: "HIP_ERROR",
}

# Every symbol the public and testing headers declare.
EXPORTED_SYMBOLS = (
    "mla_abi_version",
    "mla_last_error",
    "mla_append",
    "mla_decode_attn",
    "mla_decode_attn_append",
    "mla_decode_attn_noalloc",
    "mla_prefill_attn",
    "mla_merge",
    "mla_split_count",
    "mla_balanced_chunk",
    "mla_decode_blocks_per_cu",
    "mla_linear",
    "mla_pack_weight",
    "mla_linear_packed",
    "mla_merge_project",
    "mla_head_product",
    "mla_host_f32_to_e4m3",
    "mla_host_e4m3_to_f32",
    "mla_host_e4m3x4_to_bf16",
    "mla_host_f32_to_bf16",
    "mla_probe_read",
    "mla_probe_cache_stream",
)

_P = ctypes.c_void_p
_I32 = ctypes.c_int32
_I64 = ctypes.c_int64
_F = ctypes.c_float

_lib: Optional[ctypes.CDLL] = None


class SwamlaError(RuntimeError):
    """A non-zero status from the C-ABI; ``code`` is the SWAMLA_ERR_* value."""

    def __init__(self, code: int, msg: str):
        super().__init__(f"[{ERR_NAMES.get(code, code)}] {msg}")
        self.code = code


def _declare(lib: ctypes.CDLL) -> None:
    lib.mla_abi_version.restype = ctypes.c_int
    lib.mla_abi_version.argtypes = []
    lib.mla_last_error.restype = ctypes.c_char_p
    lib.mla_last_error.argtypes = []
    lib.mla_split_count.restype = _I32
    lib.mla_split_count.argtypes = [_I32, _I32, _I32]
    lib.mla_balanced_chunk.restype = _I32
    lib.mla_balanced_chunk.argtypes = [_P, _I32, _I32, _I32, _I32]
    lib.mla_decode_blocks_per_cu.restype = _I32
    lib.mla_decode_blocks_per_cu.argtypes = [_I32, _I32, _I32, _I32]
    lib.mla_append.restype = ctypes.c_int
    lib.mla_append.argtypes = [
        _P, _I64, _I32, _P, _P, _P, _P, _I32, _I32, _P, _P, _F, _P, _P, _I64,
        _P, _P, _P, _I64, _I64, _P, _I32, _I32, _I32, _I32, _P,
    ]
    lib.mla_decode_attn.restype = ctypes.c_int
    lib.mla_decode_attn.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64,
        _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32,
        _F, _I32, _I32, _I32, _P, _P, _P, _P, _I64, _I64, _P, _I32, _I32, _P,
    ]
    lib.mla_decode_attn_append.restype = ctypes.c_int
    lib.mla_decode_attn_append.argtypes = [
        _P, _I64, _P, _P, _F, _P,
        _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64,
        _P, _P, _P, _I64, _I64, _P, _I32, _I32, _I32, _I32, _I32,
        _F, _I32, _I32, _I32, _P, _P, _P, _P, _I64, _I64, _P, _I32, _I32, _P,
    ]
    lib.mla_decode_attn_noalloc.restype = ctypes.c_int
    lib.mla_decode_attn_noalloc.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64,
        _P, _P, _P, _I64, _I64, _P, _P, _P, _P, _I32, _I32, _I32, _I32, _I32, _I32,
        _F, _I32, _I32, _I32, _P, _I64, _I64, _P, _I32, _I32, _P,
    ]
    lib.mla_prefill_attn.restype = ctypes.c_int
    lib.mla_prefill_attn.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64, _P, _P, _I64,
        _P, _P, _P, _I64, _I64, _P, _I32, _I32, _I32, _I32, _I32, _I32,
        _F, _P, _I64, _I64, _I32, _I32, _P,
    ]
    lib.mla_merge.restype = ctypes.c_int
    lib.mla_merge.argtypes = [
        _P, _P, _P, _P, _P, _I32, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P, _P, _I64, _I64, _P, _I32, _P,
    ]
    lib.mla_pack_weight.restype = ctypes.c_int
    lib.mla_pack_weight.argtypes = [_P, _I64, _I32, _I32, _P, _I32, _P]
    lib.mla_linear_packed.restype = ctypes.c_int
    lib.mla_linear_packed.argtypes = [_P, _I64, _P, _P, _P, _I64, _I32, _I32, _I32, _P, _I32, _I32, _P]
    lib.mla_linear.restype = ctypes.c_int
    lib.mla_linear.argtypes = [
        _P, _I64, _I64, _P, _I64, _I64, _P, _I64, _P, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P,
    ]
    lib.mla_merge_project.restype = ctypes.c_int
    lib.mla_merge_project.argtypes = [
        _P, _P, _P, _I64, _I64, _P, _P, _P, _I32, _I64, _I64, _I32, _I32, _I32, _I32, _I32,
        _P, _P, _I64, _I64, _I32, _P, _I64, _I64, _I32, _P,
    ]
    lib.mla_head_product.restype = ctypes.c_int
    lib.mla_head_product.argtypes = [_P, _I64, _I64, _P, _I64, _I64, _P, _I64, _I64, _I32, _I32, _I32, _I32, _I32, _P]
    lib.mla_host_f32_to_e4m3.restype = None
    lib.mla_host_f32_to_e4m3.argtypes = [_P, _P, _I64]
    lib.mla_host_e4m3_to_f32.restype = None
    lib.mla_host_e4m3_to_f32.argtypes = [_P, _P, _I64]
    lib.mla_host_e4m3x4_to_bf16.restype = None
    lib.mla_host_e4m3x4_to_bf16.argtypes = [_P, _P, _I64]
    lib.mla_host_f32_to_bf16.restype = None
    lib.mla_host_f32_to_bf16.argtypes = [_P, _P, _I64]
    lib.mla_probe_read.restype = _I32
    lib.mla_probe_read.argtypes = [_P, _I64, _P, _I32, _P]
    lib.mla_probe_cache_stream.restype = _I32
    lib.mla_probe_cache_stream.argtypes = [_P, _P, _P, _I64, _I64, _P, _I32, _I32, _I32, _I32, _I32, _P, _P]


def lib() -> ctypes.CDLL:
    """Load the in-tree library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` "
                "(there is no CPU or eager fallback for this path)"
            )
        handle = ctypes.CDLL(LIB_PATH)
        _declare(handle)
        got = handle.mla_abi_version()
        if got != ABI_VERSION:
            raise RuntimeError(f"{LIB_NAME} ABI version {got} != expected {ABI_VERSION}")
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != 0:
        raise SwamlaError(status, lib().mla_last_error().decode())


def dtype_code(dt: torch.dtype) -> int:
    if dt == torch.float32:
        return DTYPE_F32
    if dt == torch.bfloat16:
        return DTYPE_BF16
    raise TypeError(f"unsupported model dtype {dt} (float32 or bfloat16)")


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def stream_handle(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def split_count(L: int, n_splits: int, min_chunk: int) -> int:
    return lib().mla_split_count(L, n_splits, min_chunk)
