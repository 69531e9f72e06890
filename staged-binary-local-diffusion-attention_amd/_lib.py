"""ctypes binding of the C ABI in ``include/sbda_amd.h`` (libsbda_amd.so).

The library is loaded on first use.  A missing or mismatched library raises
:class:`SBDALibraryError` -- there is no other implementation to fall back
to, by design.
"""

from __future__ import annotations

import ctypes
from pathlib import Path

LIBRARY_PATH = Path(__file__).resolve().with_name("libsbda_amd.so")
ABI_VERSION = 10

OK, ERR_VALUE, ERR_DTYPE, ERR_RUNTIME = 0, 1, 2, 3
_ERRORS = {ERR_VALUE: ValueError, ERR_DTYPE: TypeError, ERR_RUNTIME: RuntimeError}

_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_i32 = ctypes.c_int32
_f32 = ctypes.c_float
_strides = ctypes.POINTER(ctypes.c_int64)
_offs = ctypes.POINTER(ctypes.c_int32)
_fptr = ctypes.c_void_p

_SHAPE = [_i64, _i64, _i64, _i64, _i64, _i32, _offs, _i32]
_SEG = _p            # const int32_t* seg_key (device, NULL = unmasked)

# name -> (restype, argtypes); exactly the functions include/sbda_amd.h declares.
SIGNATURES = {
    "sbda_abi_version": (ctypes.c_int, []),
    "sbda_last_error": (ctypes.c_char_p, []),
    "sbda_forward": (ctypes.c_int, [_p, _strides, _p, _strides, _p, _strides, _p, _strides,
                                    _fptr, *_SHAPE, _SEG, _p]),
    "sbda_backward_workspace": (ctypes.c_int64, [*_SHAPE, _SEG]),
    "sbda_backward": (ctypes.c_int, [_p, _strides, _p, _strides, _p, _strides, _p, _strides,
                                     _fptr, _p, _strides, _p, _strides, _p, _strides, _p, _i64,
                                     *_SHAPE, _SEG, _p]),
    "sbda_forward_prologue": (ctypes.c_int, [_p, _strides, _p, _strides, _p, _strides, _p,
                                             _strides, _fptr, _fptr, _fptr, _p, _p, _f32,
                                             *_SHAPE, _SEG, _p]),
    "sbda_backward_prologue_workspace": (ctypes.c_int64, [*_SHAPE, _SEG]),
    "sbda_backward_workspace_for": (ctypes.c_int64, [_i32, *[_strides] * 7, *_SHAPE, _SEG]),
    "sbda_backward_prologue": (ctypes.c_int, [_p, _strides, _p, _strides, _p, _strides, _p,
                                              _strides, _fptr, _fptr, _fptr, _p, _p, _f32,
                                              _p, _strides, _p, _strides, _p, _strides,
                                              _fptr, _fptr, _p, _i64, *_SHAPE, _SEG, _p]),
    "sbda_noalloc_scratch_bytes": (ctypes.c_int64, []),
    "sbda_backward_prologue_noalloc": (ctypes.c_int, [_p, _strides, _p, _strides, _p, _strides,
                                                      _p, _strides, _fptr, _fptr, _fptr, _p, _p,
                                                      _f32, _p, _strides, _p, _strides, _p,
                                                      _strides, _fptr, _fptr, *_SHAPE, _SEG, _p]),
    "sbda_forward_paths": (ctypes.c_int, [_p, _strides, _p, _strides, _p, _strides, _p, _strides,
                                          _fptr, _fptr, _fptr, _p, _p, _f32,
                                          _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _i32,
                                          _SEG, _p]),
    "sbda_backward_paths_workspace": (ctypes.c_int64, [_i64, _i64, _i64, _i64, _i64, _i32, _i32,
                                                       _i32]),
    "sbda_backward_paths": (ctypes.c_int, [_p, _strides, _p, _strides, _p, _strides, _p, _strides,
                                           _fptr, _fptr, _fptr, _p, _p, _f32,
                                           _p, _strides, _p, _strides, _p, _strides,
                                           _fptr, _fptr, _p, _i64,
                                           _i64, _i64, _i64, _i64, _i64, _i32, _p, _p, _i32,
                                           _SEG, _p]),
    "sbda_rmsnorm_forward": (ctypes.c_int, [_p, _p, _p, _p, _fptr, _fptr, _i64, _i64, _i32, _f32,
                                            _p]),
    "sbda_rmsnorm_backward_workspace": (ctypes.c_int64, [_i64, _i64, _i32]),
    "sbda_rmsnorm_backward": (ctypes.c_int, [_p, _p, _fptr, _fptr, _p, _p, _fptr, _p, _i64, _i64,
                                             _i64, _i32, _p]),
    "sbda_swiglu_forward": (ctypes.c_int, [_p, _p, _i64, _i64, _i32, _p]),
    "sbda_swiglu_backward": (ctypes.c_int, [_p, _p, _p, _i64, _i64, _i32, _p]),
    "sbda_swiglu_gemm_supported": (ctypes.c_int, [_i64, _i64, _i64, _i32]),
    "sbda_swiglu_gemm_forward": (ctypes.c_int, [_p, _p, _fptr, _p, _i64, _i64, _i64, _i32, _p]),
    "sbda_rope_table": (ctypes.c_int, [_p, _p, ctypes.POINTER(ctypes.c_float), _i64, _i64, _p]),
}


class SBDALibraryError(RuntimeError):
    """The HIP library is not built, not loadable, or from another ABI."""


_LIB: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIBRARY_PATH.exists():
        raise SBDALibraryError(
            f"{LIBRARY_PATH} is not built; run `python __graft_entry__.py` "
            "(or build.py) on a machine with ROCm's hipcc")
    try:
        lib = ctypes.CDLL(str(LIBRARY_PATH))
    except OSError as exc:
        raise SBDALibraryError(f"cannot load {LIBRARY_PATH}: {exc}") from exc
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.sbda_abi_version() != ABI_VERSION:
        raise SBDALibraryError(
            f"{LIBRARY_PATH} has ABI {lib.sbda_abi_version()}, expected {ABI_VERSION}; rebuild it")
    _LIB = lib
    return lib


def check(rc: int) -> None:
    """Raise the Python error class of a non-zero C ABI status."""
    if rc == OK:
        return
    msg = (load().sbda_last_error() or b"").decode(errors="replace")
    raise _ERRORS.get(rc, RuntimeError)(msg or f"SBDA error code {rc}")


def strides(t) -> ctypes.Array:
    return (ctypes.c_int64 * 4)(*t.stride())


def offsets_array(offsets) -> ctypes.Array:
    return (ctypes.c_int32 * len(offsets))(*offsets)
