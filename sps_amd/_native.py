"""ctypes binding of libsps_attn.so (the C ABI declared in include/sps_attn.h).

The library is loaded lazily on first use and the load fails loudly: there is no fallback path.
"""

from __future__ import annotations

import ctypes as C
import threading
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libsps_attn.so"

SPS_OK = 0
SPS_E_INVALID = 1
SPS_E_UNSUPPORTED = 2
SPS_E_WORKSPACE = 3
SPS_E_HIP = 4

DTYPE_BF16 = 0
DTYPE_F16 = 1
DTYPE_F32 = 2
DTYPE_I32 = 3
DTYPE_I64 = 4
DTYPE_U8 = 5

BWD_DQ = 1
BWD_DKDV = 2
BWD_REUSE_LAYOUT = 4

FAMILY_FULL = 0
FAMILY_SPS = 1
FAMILY_REVERSE_SPS = 2

EXPORTED_SYMBOLS = (
    "sps_version",
    "sps_last_error",
    "sps_attn_workspace_bytes",
    "sps_attn_fwd",
    "sps_attn_bwd",
    "sps_attn_bwd_pass",
    "sps_attn_mask",
    "sps_decode_workspace_bytes",
    "sps_decode",
    "sps_decode_static",
    "sps_kv_update",
    "sps_decode_kv_update_workspace_bytes",
    "sps_decode_kv_update",
    "sps_rope_qkv",
    "sps_prefill_to_decode",
    "sps_document_ids",
)

_i32 = C.c_int
_i64 = C.c_int64
_p = C.c_void_p
_pi64 = C.POINTER(C.c_int64)
_pi32 = C.POINTER(C.c_int)
_f32 = C.c_float
_sz = C.c_size_t

_SIGNATURES = {
    "sps_version": (C.c_char_p, []),
    "sps_last_error": (_i32, [C.c_char_p, _sz]),
    "sps_attn_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "sps_attn_fwd": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32, _i32]
        + [_p, _pi64] * 4
        + [_p]  # lse
        + [_p, _i32, _i64]  # docs
        + [_f32, _i32, _i32, _i32]
        + [_p, _sz, _p],
    ),
    "sps_attn_bwd": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32, _i32]
        + [_p, _pi64] * 5
        + [_p]  # lse
        + [_p, _pi64] * 3
        + [_p, _i32, _i64]
        + [_f32, _i32, _i32, _i32]
        + [_p, _sz, _p],
    ),
    "sps_attn_bwd_pass": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32, _i32, _i32]
        + [_p, _pi64] * 5
        + [_p]  # lse
        + [_p, _pi64] * 3
        + [_p, _i32, _i64]
        + [_f32, _i32, _i32, _i32]
        + [_p, _sz, _p],
    ),
    "sps_attn_mask": (
        _i32,
        [_i32, _i32, _i32, _p, _i32, _i64, _i32, _i32, _i32, _i32, _p, _p, _sz, _p],
    ),
    "sps_decode_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _pi64]),
    "sps_decode": (
        _i32,
        [_i32, _i32, _i32, _i32, _p, _i32, _pi64, _i32, _i32]
        + [C.POINTER(_p), _pi64, C.POINTER(_p), _pi64, C.POINTER(_p), _pi32, _pi32, _pi64]
        + [_i32, C.POINTER(_p), C.POINTER(_p), _i32, _pi64, _pi32]
        + [_f32, _p, _pi64, _p, _sz, _p],
    ),
    "sps_decode_static": (
        _i32,
        [_i32, _i32, _i32, _i32, _p, _i32, _pi64, _i32, _i32]
        + [C.POINTER(_p), _pi64, C.POINTER(_p), _pi64, C.POINTER(_p), _pi32, _pi32, _pi64]
        + [_i32, C.POINTER(_p), C.POINTER(_p), _i32, _pi64, _pi32]
        + [_f32, _p, _pi64, _p],
    ),
    "sps_kv_update": (
        _i32,
        [_i32, _i32, _i32, _i32]
        + [_p, _p, _pi64, _i32, _i32, _p, _p, _pi64]  # ring
        + [_p, _p, _pi64, _i32, _p, _pi64, _i32]  # retained, length dtype
        + [_i32, _p, _p, _p, _p, _pi64]  # new K/V
        + [_p, _i32, _i64, _p],
    ),
    "sps_decode_kv_update_workspace_bytes": (_sz, [_i32, _i32, _i32, _i32, _i32, _i32, _pi64]),
    "sps_decode_kv_update": (
        _i32,
        [_i32, _i32, _i32, _i32, _p, _i32, _pi64, _i32, _i32]
        + [C.POINTER(_p), _pi64, C.POINTER(_p), _pi64, C.POINTER(_p), _pi32, _pi32, _pi64]
        + [_i32, C.POINTER(_p), C.POINTER(_p), _i32, _pi64, _pi32]
        + [_f32, _p, _pi64]
        + [_p, _p, _pi64, _i32, _i32, _p, _p, _pi64]  # ring
        + [_p, _p, _pi64, _i32, _p, _pi64, _i32]  # retained, length dtype
        + [_i32, _p, _p, _p, _p, _pi64]  # new K/V
        + [_p, _i32, _i64]  # active
        + [_p, _sz, _p],
    ),
    "sps_rope_qkv": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32]
        + [_p, _pi64] * 3
        + [_p, _pi64, _i32]
        + [_p, _pi64] * 3
        + [_p],
    ),
    "sps_prefill_to_decode": (
        _i32,
        [_i32, _i32, _i32, _i32, _i32, _p, _pi64, _p, _pi64, _i32, _i32, _p, _i64, _i32]
        + [_p, _p, _pi64, _i32, _i32, _p, _p, _pi64]  # ring
        + [_p, _p, _pi64, _i32, _p, _pi64, _i32]  # retained, length dtype
        + [_p],
    ),
    "sps_document_ids": (_i32, [_i32, _i32, _p, _i32, _i64, _i64, _i64, _i32, _p, _i32, _i64, _p, _p]),
}

_lib = None
_lock = threading.Lock()


class NativeError(RuntimeError):
    """An entry point of libsps_attn.so returned an error status."""

    def __init__(self, func: str, code: int, message: str):
        super().__init__(f"{func} failed with status {code}: {message}")
        self.code = code


def lib() -> C.CDLL:
    """Returns the loaded library, loading it on first use."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise ImportError(
                    f"sps_amd: native library {LIB_PATH} is missing; build it with "
                    "`python -m sps_amd.build` (there is no fallback implementation)"
                )
            handle = C.CDLL(str(LIB_PATH))
            for name, (res, args) in _SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def last_error() -> str:
    buf = C.create_string_buffer(1024)
    lib().sps_last_error(buf, len(buf))
    return buf.value.decode(errors="replace")


def check(func: str, status: int) -> None:
    if status != SPS_OK:
        raise NativeError(func, status, last_error())


def i64_array(values) -> C.Array:
    vals = list(values)
    return (C.c_int64 * max(len(vals), 1))(*vals)


_CONST_CACHE: dict = {}


def _const_array(ctype, values: tuple) -> C.Array:
    """A ctypes array of `values`, cached by value, for the array arguments of per-call host paths
    (strides, sizes, pointers that stay the same from call to call, such as KV caches): the native
    entry points only read these arrays during the call and nothing writes them, so equal tuples can
    share one array (the cache is emptied past 1024 entries)."""
    key = (ctype, values)
    arr = _CONST_CACHE.get(key)
    if arr is None:
        if len(_CONST_CACHE) >= 1024:
            _CONST_CACHE.clear()
        arr = _CONST_CACHE[key] = (ctype * max(len(values), 1))(*values)
    return arr


def i64_const(values: tuple) -> C.Array:
    """i64_array of a tuple of ints, cached by value (see _const_array)."""
    return _const_array(C.c_int64, values)


def i32_const(values: tuple) -> C.Array:
    """i32_array of a tuple of ints, cached by value (see _const_array)."""
    return _const_array(C.c_int, values)


def ptr_const(values: tuple) -> C.Array:
    """ptr_array of a tuple of addresses (ints or None for null), cached by value (see _const_array)."""
    return _const_array(C.c_void_p, values)


def i32_array(values) -> C.Array:
    vals = list(values)
    return (C.c_int * max(len(vals), 1))(*vals)


def ptr_array(values) -> C.Array:
    vals = [v if v is not None else 0 for v in values]
    return (C.c_void_p * max(len(vals), 1))(*vals)
