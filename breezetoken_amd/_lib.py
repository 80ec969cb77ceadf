"""ctypes binding of libbreezetoken_amd.so (the C ABI in include/breezetoken_amd.h).

The library is loaded from this package directory only.  There is no fallback:
if it is missing, ``lib()`` raises and every operator that needs it fails.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libbreezetoken_amd.so"

BT_OK = 0
BT_EINVAL = -22
BT_ENOTSUP = -95
BT_ENOSPC = -28
BT_DTYPE_F32 = 0
BT_DTYPE_BF16 = 1
BT_NOALLOC_SCRATCH_BYTES = 8 << 20

_c_i32 = ctypes.c_int32
_c_i64 = ctypes.c_int64
_c_f32 = ctypes.c_float
_vp = ctypes.c_void_p

# name -> (restype, argtypes); the order mirrors include/breezetoken_amd.h.
SIGNATURES: dict[str, tuple[object, list[object]]] = {
    "bt_version": (ctypes.c_int, []),
    "bt_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "bt_decode_tile_tokens": (_c_i32, []),
    "bt_decode_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32]),
    "bt_decode_pick_splits": (_c_i32, [_c_i32, _c_i32, _c_i32]),
    "bt_gqa_decode_split": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_f32, _vp, _vp, _vp],
    ),
    "bt_gqa_decode_combine": (
        ctypes.c_int,
        [_vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32, _vp, _vp, _c_i32, _vp, _c_i32, _c_i64, _vp],
    ),
    "bt_gqa_decode": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_f32, _vp, _c_i64, _vp, _c_i32, _c_i64, _vp],
    ),
    "bt_gqa_decode_noalloc": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32,
         _c_i32, _c_i32, _c_i32, _c_f32, _vp, _c_i32, _c_i64, _vp],
    ),
    "bt_ragged_plan": (
        _c_i32,
        [_vp, _c_i32, _c_i32, _vp, _c_i32, _vp, _vp, _vp],
    ),
    "bt_ragged_plan_device": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i32, _vp, _c_i32, _vp, _vp, _vp, _vp],
    ),
    "bt_gqa_decode_ragged": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i64, _vp, _vp, _c_i64, _c_i64, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_i32,
         _vp, _c_i32, _vp, _vp, _c_i32, _c_f32, _vp, _c_i64, _vp, _c_i32, _c_i64, _vp],
    ),
    "bt_prefill_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32]),
    "bt_prefill_split_workspace_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "bt_gqa_prefill": (
        ctypes.c_int,
        [_vp, _c_i32, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
         _c_f32, _vp, _c_i64, _vp, _c_i32, _c_i64, _c_i64, _vp],
    ),
    "bt_prefill_partials_bytes": (_c_i64, [_c_i32, _c_i32, _c_i32, _c_i32, _c_i32]),
    "bt_gqa_prefill_cached": (
        ctypes.c_int,
        [_vp, _c_i32, _vp, _vp, _c_i64, _c_i64, _c_i64, _c_i64, _c_i32, _c_i32, _c_i32, _c_i32, _c_i32,
         _c_f32, _vp, _c_i64, _c_i32, _c_i32, _vp, _c_i64, _vp, _c_i32, _c_i64, _c_i64, _vp],
    ),
    "bt_rms_norm_rope": (
        ctypes.c_int,
        [_vp, _c_i64, _c_i32, _c_i32, _vp, _c_f32, _vp, _vp, _vp, _c_i32, _c_i32, _vp, _c_i64, _vp],
    ),
    "bt_attn_prep": (
        ctypes.c_int,
        [_vp, _c_i32, _c_i32, _c_i32, _vp, _vp, _c_f32, _vp, _vp, _vp, _c_i32, _c_i32, _vp, _c_i32,
         _vp, _vp, _c_i64, _c_i64, _c_i32, _vp],
    ),
    "bt_gdn_decode": (
        ctypes.c_int,
        [_vp, _vp, _vp, _vp, _vp, _vp, _c_i32, _c_i32, _c_i32, _c_f32, _c_f32, _vp, _vp],
    ),
    "bt_gemv_workspace_bytes": (_c_i64, [_c_i32, _c_i32]),
    "bt_gemv_bf16": (
        ctypes.c_int,
        [_vp, _vp, _c_i64, _c_i32, _c_i32, _vp, _vp, _c_i64, _vp],
    ),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class BreezeTokenAmdError(RuntimeError):
    """A C-ABI call returned a non-zero code."""

    def __init__(self, fn: str, code: int, message: str) -> None:
        super().__init__(f"{fn} failed with code {code}: {message}")
        self.fn = fn
        self.code = code


def lib() -> ctypes.CDLL:
    """Load (once) and return the HIP library; raise if it has not been built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.is_file():
                raise RuntimeError(
                    f"{LIB_PATH.name} is missing; build it with `python -m breezetoken_amd.build`"
                )
            handle = ctypes.CDLL(str(LIB_PATH))
            for name, (restype, argtypes) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = restype
                fn.argtypes = argtypes
            _lib = handle
    return _lib


def strerror(code: int) -> str:
    return lib().bt_strerror(code).decode()


def check(fn: str, code: int) -> None:
    if code != BT_OK:
        raise BreezeTokenAmdError(fn, code, strerror(code))
