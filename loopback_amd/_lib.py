"""ctypes binding of libloopback_read.so (the C ABI declared in include/loopback_read.h).

Loading fails loudly: a missing or stale library raises ImportError at import time, and every entry point that
returns a nonzero code raises RuntimeError with the library's own message. There is no fallback path.
"""
from __future__ import annotations

import ctypes
import os

import torch  # noqa: F401  -- first: the library must bind to the HIP runtime torch already loaded (same soname)

from . import build as _build

ABI_VERSION = 16
F32, BF16, F16 = 0, 1, 2
MAX_SOURCES = 64
MAX_WIDTH = 8192
MAX_QUERIES = 64
ANY_MAX_SOURCES = 1024   # the *_any entry points (device address arrays)

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int
_f32 = ctypes.c_float
_u64p = ctypes.POINTER(ctypes.c_uint64)

# name -> (restype, argtypes); one line per declaration of include/loopback_read.h
SIGNATURES = {
    "ldr_abi_version": (_i32, []),
    "ldr_strerror": (ctypes.c_char_p, [_i32]),
    "ldr_row_layout": (_i32, [_i64, ctypes.POINTER(_i32), ctypes.POINTER(_i32)]),
    "ldr_read_bwd1_parts": (_i64, [_i64, _i64]),
    "ldr_rstd_fwd": (_i32, [_c_void_p, _c_void_p, _i64, _i64, _f32, _i32, _c_void_p]),
    "ldr_rstd_bwd": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ldr_write_dots": (_i32, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64,
                              _c_void_p, _i64, _i64, _i64, _f32, _i32, _c_void_p]),
    "ldr_query_parts_elems": (_i64, [_i64, _i64]),
    "ldr_split_queries": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "ldr_dots_online": (_i32, [_u64p, _i64, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32, _c_void_p]),
    "ldr_read_fwd": (_i32, [_u64p, _u64p, _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _f32, _c_void_p, _i64,
                            _c_void_p, _i64, _f32, _f32, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i32,
                            _c_void_p]),
    "ldr_read_fwd_online": (_i32, [_u64p, _u64p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _f32,
                                   _c_void_p, _i64, _c_void_p, _i64, _f32, _f32, _c_void_p, _c_void_p, _c_void_p,
                                   _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ldr_read_bwd1": (_i32, [_u64p, _u64p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p,
                             _c_void_p, _i64, _c_void_p, _i64, _f32, _f32, _c_void_p, _i64, _u64p, _i32, _c_void_p,
                             _i64, _c_void_p, _i64, _c_void_p, _c_void_p, _f32, _i64, _i64, _i32, _c_void_p]),
    "ldr_read_bwd1_noalloc": (_i32, [_u64p, _u64p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                     _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _f32, _f32, _c_void_p, _i64, _u64p,
                                     _i32, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _f32, _i64, _i64, _i32,
                                     _c_void_p]),
    "ldr_reduce_rows": (_i32, [_c_void_p, _i64, _i64, _c_void_p, _c_void_p]),
    "ldr_read_bwd2_list": (_i32, [_u64p, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32,
                                  _c_void_p]),
    "ldr_dv_assemble": (_i32, [_u64p, _u64p, _u64p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _f32, _i32,
                               _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ldr_blend_sum": (_i32, [_u64p, _i64, _f32, _i32, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    # the any-shape entry points: per-source addresses in device arrays (passed as device addresses)
    "ldr_read_fwd_any": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _f32,
                                _c_void_p, _i64, _c_void_p, _i64, _f32, _f32, _c_void_p, _c_void_p, _c_void_p,
                                _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ldr_read_bwd1_any": (_i32, [_c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
                                 _c_void_p, _c_void_p, _i64, _c_void_p, _i64, _f32, _f32, _c_void_p, _i64, _c_void_p,
                                 _i32, _c_void_p, _i64, _c_void_p, _i64, _i64, _c_void_p, _c_void_p, _f32, _i64, _i64,
                                 _i32, _c_void_p]),
    "ldr_dv_assemble_any": (_i32, [_c_void_p, _c_void_p, _c_void_p, _i64, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
                                   _f32, _i32, _c_void_p, _c_void_p, _i64, _i64, _i32, _c_void_p]),
    "ldr_read_bwd2_list_any": (_i32, [_c_void_p, _i64, _i32, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i32,
                                      _c_void_p]),
    "ldr_blend_sum_any": (_i32, [_c_void_p, _i64, _f32, _i32, _c_void_p, _i64, _i64, _i32, _c_void_p]),
}


def _load() -> ctypes.CDLL:
    path = os.environ.get("LOOPBACK_READ_LIB", _build.LIB)
    if not os.path.exists(path):
        raise ImportError(f"loopback_read: {path} is not built (run `python -m loopback_amd.build`); "
                          "the HIP read has no fallback")
    try:
        lib = ctypes.CDLL(path)
    except OSError as e:
        raise ImportError(f"loopback_read: cannot load {path}: {e}") from e
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)          # AttributeError -> the library is stale
        fn.restype, fn.argtypes = res, args
    if lib.ldr_abi_version() != ABI_VERSION:
        raise ImportError(f"loopback_read: {path} has ABI {lib.ldr_abi_version()}, expected {ABI_VERSION}; rebuild")
    return lib


LIB = _load()
PATH = os.environ.get("LOOPBACK_READ_LIB", _build.LIB)


def check(code: int, what: str) -> None:
    if code != 0:
        msg = LIB.ldr_strerror(code).decode()
        raise RuntimeError(f"{what}: {msg} (code {code})")


def u64_array(values) -> ctypes.Array:
    """A host array of device addresses (ints) for a per-source argument."""
    vals = values if isinstance(values, list) else list(values)
    return (ctypes.c_uint64 * max(1, len(vals)))(*vals)


def row_layout(d: int) -> tuple[int, int]:
    vpt, tpr = _i32(), _i32()
    check(LIB.ldr_row_layout(d, ctypes.byref(vpt), ctypes.byref(tpr)), f"row layout d={d}")
    return vpt.value, tpr.value


def bwd1_parts(n_tok: int, d: int) -> int:
    return int(LIB.ldr_read_bwd1_parts(n_tok, d))
