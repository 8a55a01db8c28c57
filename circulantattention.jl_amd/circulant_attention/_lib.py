"""ctypes binding of libcircatt.so (the C ABI declared in include/circatt.h).

The library is required: importing this module raises if it has not been
built (``python circulantattention.jl_amd/build.py``).  There is no CPU or
PyTorch fallback for any operation.
"""
from __future__ import annotations

import ctypes
import os

# torch bundles its own HIP runtime under the soname libamdhip64.so.7, the
# soname libcircatt.so links against.  Loaded after torch, libcircatt binds to
# that already-loaded runtime, so one HIP runtime serves both; loaded first,
# it would pull in /opt/rocm's copy and torch would then load a second one,
# and two runtimes in one process do not share the device (the second reports
# none).  So torch is imported before the library is opened.
import torch  # noqa: F401

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get(
    "CIRCATT_LIB", os.path.join(os.path.dirname(_HERE), "libcircatt.so"))

OK = 0
ERR_INVALID = -1
ERR_UNSUPPORTED = -2
ERR_HIP = -3

DOT = 0
DISTANCE = 1
F32 = 0
C32 = 1
CHANNELS_LAST = 16  # OR-ed into dtype of the fused entry points

MATH_SPLIT_F16 = 0
MATH_F32 = 1

_i32 = ctypes.c_int32
_int = ctypes.c_int
_i64 = ctypes.c_int64
_f32 = ctypes.c_float
_p = ctypes.c_void_p

# name -> (restype, argtypes); the exported C ABI, one entry per declaration
SIGNATURES = {
    "circatt_version": (_int, []),
    "circatt_last_error": (ctypes.c_char_p, []),
    "circatt_set_math": (_int, [_int]),
    "circatt_get_math": (_int, []),
    "circatt_pattern": (_int, [_int, _i64, _i64, _i32, _i64, _p, _p, _p]),
    "circatt_similarity": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _f32, _p, _p,
                                  _p, _p]),
    "circatt_softmax": (_int, [_i64, _i64, _p, _p, _p]),
    "circatt_softmax_bwd": (_int, [_i64, _i64, _p, _p, _p, _p]),
    "circatt_apply": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _p, _p, _p, _p]),
    "circatt_similarity_bwd": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _f32, _p,
                                      _p, _p, _p, _p, _p]),
    "circatt_rowsum": (_int, [_int, _i64, _i64, _i32, _i64, _p, _p, _p]),
    "circatt_colsum": (_int, [_int, _i64, _i64, _i32, _i64, _p, _p, _p]),
    "circatt_axpby": (_int, [_i64, _i64, _p, _f32, _p, _p, _f32, _p, _p, _p]),
    "circatt_batch_dot_workspace_bytes": (_i64, [_i64, _i64]),
    "circatt_batch_dot": (_int, [_i64, _i64, _p, _p, _p, _p, _i64, _p]),
    "circatt_fused_fwd": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _i64, _p, _p,
                                 _p, _p, _p, _p]),
    "circatt_fused_bwd_workspace_bytes": (_i64, [_int, _i64, _i64, _i64, _i64]),
    "circatt_fused_bwd": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _i64, _p, _p,
                                 _p, _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "circatt_fused_bwd_dq": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _i64, _p,
                                    _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "circatt_fused_bwd_dkdv": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _i64, _p,
                                      _p, _p, _p, _p, _p, _p, _p, _i64, _p]),
    "circatt_fused_bwd_noalloc_max_rows": (_i64, []),
    "circatt_fused_bwd_noalloc": (_int, [_int, _int, _int, _i64, _i64, _i32, _i64, _i64, _i64,
                                         _p, _p, _p, _p, _p, _p, _p, _p, _p, _p]),
    "circatt_fill": (_int, [_p, _i64, _f32, _p]),
    "circatt_copy_blocks": (_int, [_p, _p, _i64, _i64, _i64, _i64, _i64, _i64, _i64, _p]),
    "circatt_sum_middle": (_int, [_p, _p, _i64, _i64, _i64, _p]),
    "circatt_count_unequal": (_int, [_int, _i64, _p, _p, _p, _p]),
    "circatt_malloc": (_int, [ctypes.POINTER(_p), _i64]),
    "circatt_free": (_int, [_p]),
    "circatt_memcpy": (_int, [_p, _p, _i64, _int]),
    "circatt_stream_synchronize": (_int, [_p]),
}


class CircAttError(RuntimeError):
    """A HIP runtime failure reported by libcircatt."""


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"libcircatt.so not found at {LIB_PATH}; build it with "
            "`python circulantattention.jl_amd/build.py` (no fallback exists)")
    lib = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def check(rc: int, what: str = "") -> None:
    """Raise the Python counterpart of a libcircatt error code."""
    if rc == OK:
        return
    msg = lib.circatt_last_error().decode() or what
    if rc == ERR_INVALID:
        raise AssertionError(msg)  # the reference raises from @assert
    if rc == ERR_UNSUPPORTED:
        raise NotImplementedError(msg)
    raise CircAttError(msg)
