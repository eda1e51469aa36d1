"""
ctypes binding of the C ABI declared in include/pagedkv.h.

The library is built in-tree (``python -m llm_serving_layer_amd.build``) into
``_native/libpagedkv.so``. There is no fallback: if it cannot be loaded,
``load()`` raises and every caller of the GPU path fails loudly.
"""

from __future__ import annotations

import ctypes as C
import os
from pathlib import Path

# PKV_LIBRARY selects another build of the same library (e.g. a tuning variant).
LIB_PATH = Path(os.environ.get("PKV_LIBRARY") or
                Path(__file__).resolve().parent / "_native" / "libpagedkv.so")
ABI_VERSION = 11

DTYPE_F16, DTYPE_BF16, DTYPE_F32 = 0, 1, 2
DECODE_SCRATCH_BYTES = 64 * 1024 * 1024   # PKV_DECODE_SCRATCH_BYTES
OK, ERR_INVALID, ERR_RANGE, ERR_HIP, ERR_CAPACITY = 0, 1, 2, 3, 4
STATUS_BAD_SLOT, STATUS_BAD_PAGE, STATUS_BAD_BLOCK = 1, 2, 4

_p, _i32, _i64, _f32 = C.c_void_p, C.c_int32, C.c_int64, C.c_float

# name -> (restype, argtypes); one entry per declaration in include/pagedkv.h
SIGNATURES = {
    "pkv_abi_version": (C.c_int, []),
    "pkv_last_error": (C.c_char_p, []),
    "pkv_append_kv": (C.c_int, [_p, _p, _i64, _p, _p, _p, _i64, _i32, _i32, _i32, _p, _p]),
    "pkv_plan_decode": (C.c_int, [_p, _p, _p, _p, _i32, _i32, _i64, _i32, _i32, _i32, _p, _i64,
                                  _p, _p, _p, _p]),
    "pkv_decode_workgroups": (C.c_int, [_i32, _i32, _i32, _i32, _i32]),
    "pkv_decode_workspace_bytes": (C.c_int64, [_i32, _i32, _i32, _i32, _i32]),
    "pkv_decode_fast_path": (C.c_int, [_i32, _i32, _i32, _i32, _i32, _i32]),
    "pkv_attend_decode": (C.c_int, [_p, _p, _p, _p, _i64, _p, _p, _p, _i32, _i32, _i32, _i32,
                                    _i32, _f32, _i32, _p, _i32, _i32, _i32, _p, _p, _p, _p,
                                    _i64, _p, _p]),
    "pkv_attend_decode_noalloc": (C.c_int, [_p, _p, _p, _p, _i64, _p, _p, _p, _i32, _i32, _i32,
                                            _i32, _i32, _f32, _i32, _p, _i32, _i32, _i32, _p,
                                            _p, _p, _p, _p]),
    "pkv_plan_prefill": (C.c_int, [_p, _p, _p, _p, _i32, _i32, _i32, _p, _i64, _p]),
    "pkv_prefill_q_tile": (C.c_int, [_i32, _i32, _i32, _i32, _i32]),
    "pkv_attend_prefill": (C.c_int, [_p, _p, _p, _p, _i64, _p, _p, _p, _p, _p, _i32, _i32,
                                     _i32, _i32, _i32, _i32, _f32, _i32, _p, _i32, _i32, _p,
                                     _p]),
    "pkv_copy_blocks": (C.c_int, [_p, _i32, _i64, _i64, _i64, _p, _p, _i32, _p, _p]),
    "pkv_gather_blocks": (C.c_int, [_p, _i32, _i64, _i64, _i64, _p, _i32, _p, _p, _p]),
    "pkv_scatter_blocks": (C.c_int, [_p, _i32, _i64, _i64, _i64, _p, _i32, _p, _p, _p]),
    "pkv_argmax_rows": (C.c_int, [_p, _i64, _i64, _i64, _i32, _p, _p]),
    "pkv_upload_pinned": (C.c_int, [_p, _p, _i64, _p]),
}

_LIB = None
_REASON = None


class NativeError(RuntimeError):
    """A non-zero return from the library that is not an argument error."""


def load():
    """Load the library once; raise RuntimeError with the reason if impossible."""
    global _LIB, _REASON
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        _REASON = (f"{LIB_PATH} is not built; run `python -m llm_serving_layer_amd.build` "
                   "(hipcc for gfx950)")
        raise RuntimeError(_REASON)
    try:
        lib = C.CDLL(str(LIB_PATH))
    except OSError as exc:
        _REASON = f"cannot load {LIB_PATH}: {exc}"
        raise RuntimeError(_REASON) from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    ver = lib.pkv_abi_version()
    if ver != ABI_VERSION:
        _REASON = f"{LIB_PATH} has ABI {ver}, this package expects {ABI_VERSION}; rebuild"
        raise RuntimeError(_REASON)
    _LIB = lib
    return lib


def available() -> bool:
    try:
        load()
        return True
    except RuntimeError:
        return False


def reason() -> str | None:
    return None if available() else _REASON


def check(rc: int, what: str) -> None:
    """Translate a return code into the reference's exception types."""
    if rc == OK:
        return
    msg = f"{what}: {load().pkv_last_error().decode(errors='replace')}"
    if rc in (ERR_INVALID, ERR_CAPACITY):
        raise ValueError(msg)
    if rc == ERR_RANGE:
        raise IndexError(msg)
    raise NativeError(msg)
