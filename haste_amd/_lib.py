"""ctypes binding of libhaste_ffi.so (the gfx950 HIP library, C ABI in include/haste_ffi.h).

There is no fallback: if the library is missing or cannot be loaded, every
entry point raises.  Build it with ``python -c "import __graft_entry__ as g; g.build()"``
or ``make -C haste_amd``.
"""
from __future__ import annotations

import ctypes
import os
import threading

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libhaste_ffi.so")

# Status codes and enums, mirroring include/haste_ffi.h.
HASTE_OK = 0
HASTE_ERR_INVALID_ARG = -1
HASTE_ERR_UNSUPPORTED = -2
HASTE_ERR_WORKSPACE = -3
HASTE_ERR_HIP = -4

DTYPE_BF16, DTYPE_F16, DTYPE_F32 = 0, 1, 2
DTYPE_F8E4M3, DTYPE_F8E5M2 = 3, 4  # SR outputs and SGD weights only
PRUNE_THRESHOLD, PRUNE_FRACTION, PRUNE_GLOBAL_FRACTION = 0, 1, 2
SCORE_MEAN, SCORE_MAX = 0, 1
REGROW_RANDOM, REGROW_UNUSED = 0, 1
INIT_ZERO, INIT_RANDOM = 0, 1



class SgdTensor(ctypes.Structure):
    """haste_sgd_tensor of include/haste_ffi.h."""
    _fields_ = [("w", ctypes.c_void_p), ("g", ctypes.c_void_p), ("m", ctypes.c_void_p),
                ("n", ctypes.c_int64), ("offset0", ctypes.c_uint64)]


# Every symbol declared in include/haste_ffi.h: name -> (restype, argtypes).
_P = ctypes.c_void_p
_I64 = ctypes.c_int64
_I32 = ctypes.c_int32
_U64 = ctypes.c_uint64
_F32 = ctypes.c_float
SIGNATURES = {
    "haste_last_error": (ctypes.c_char_p, []),
    "haste_abi_version": (ctypes.c_int, []),
    "haste_ffi_forward": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _I64, _I64, _I64, _I64, _I64,
                                         _I64, _I32, _P]),
    "haste_ffi_forward_f16_f32out": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _I64, _I64, _I64,
                                                    _I64, _I64, _I64, _P]),
    "haste_ffi_forward_bce_workspace_size": (_I64, [_I64, _I64, _I64]),
    "haste_ffi_forward_bce": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _I64, _P, _I64, _P, _P, _P,
                                             _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P]),
    "haste_ffi_forward_bce_noalloc": (ctypes.c_int, [_P, _P, _I64, _P, _P, _P, _I64, _P, _I64, _P,
                                                     _P, _I64, _I64, _I64, _I64, _I64, _I32, _P]),
    "haste_ffi_bwd_features_workspace_size": (_I64, [_I64, _I64, _I64, _I64, _I64, _I32]),
    "haste_ffi_bwd_features_config": (ctypes.c_int, [_I64, _I64, _I64, _I64, _I64, _I32, _P]),
    "haste_ffi_bwd_features_set_build": (ctypes.c_int, [_I32]),
    "haste_ffi_bwd_features_plan": (ctypes.c_int, [_P, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                                   _I32, _P]),
    "haste_ffi_bwd_features": (ctypes.c_int, [_P, _P, _P, _I64, _P, _P, _I64, _I64, _I64, _I64,
                                              _I64, _I64, _I32, _I32, _P]),
    "haste_ffi_bwd_features_sr": (ctypes.c_int, [_P, _P, _P, _I64, _P, _U64, _P, _I64, _I64, _I64,
                                                 _I64, _I64, _I64, _I32, _I32, _P]),
    "haste_ffi_bwd_features_partials": (ctypes.c_int, [_P, _P, _P, _I64, _P, _I64, _I64, _I64,
                                                       _I64, _I64, _I64, _I32, _I32, _P]),
    "haste_ffi_bwd_weights": (ctypes.c_int, [_P, _P, _I64, _P, _I64, _P, _I32, _P, _I32, _I64,
                                             _I64, _I64, _I64, _I64, _I32, _P]),
    "haste_ffi_bwd_weights_dx": (ctypes.c_int, [_P, _P, _I64, _P, _I64, _P, _I32, _P, _I32, _P,
                                                _U64, _P, _I64, _I64, _I64, _I64, _I64, _I64,
                                                _I32, _P]),
    "haste_ffi_bwd_weights_sgd": (ctypes.c_int, [_P, _P, _I64, _P, _I64, _P, _P, _P, _P, _P, _I32,
                                                 _P, _I32, _F32, _F32, _F32, _I32, _I32, _U64,
                                                 _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32,
                                                 _P]),
    "haste_ffi_bwd_weights_sgd_dx": (ctypes.c_int, [_P, _P, _I64, _P, _I64, _P, _P, _P, _P, _F32,
                                                    _F32, _F32, _I32, _I32, _U64, _P, _U64, _P,
                                                    _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P]),
    "haste_ffi_bwd_weights_sgd_dx_dev_seed": (ctypes.c_int, [_P, _P, _I64, _P, _I64, _P, _P, _P,
                                                             _P, _F32, _F32, _F32, _I32, _I32,
                                                             _P, _P, _U64, _P, _I64, _I64, _I64,
                                                             _I64, _I64, _I64, _I32, _P]),
    "haste_sgd_sr_step_wt": (ctypes.c_int, [_P, _P, _I32, _P, _F32, _F32, _F32, _I32, _I32, _U64,
                                            _P, _I64, _I64, _I64, _I64, _I64, _I64, _I32, _P]),
    "haste_sgd_sr_step_wt_bias": (ctypes.c_int, [_P, _P, _I32, _P, _P, _P, _I32, _P, _F32, _F32,
                                                 _F32, _I32, _I32, _U64, _P, _I64, _I64, _I64,
                                                 _I64, _I64, _I64, _I32, _P]),
    "haste_sr_round_bf16": (ctypes.c_int, [_P, _P, _I64, _U64, _U64, _P]),
    "haste_sr_round": (ctypes.c_int, [_P, _P, _I32, _I64, _U64, _U64, _P]),
    "haste_sgd_sr_step_f8": (ctypes.c_int, [_P, _I32, _P, _I32, _P, _I64, _F32, _F32, _F32,
                                            _I32, _I32, _U64, _U64, _P]),
    "haste_sr_words_fold": (ctypes.c_int, [_P, _I64, _U64, _P]),
    "haste_sgd_sr_step": (ctypes.c_int, [_P, _P, _I32, _P, _I64, _F32, _F32, _F32, _I32, _I32,
                                         _U64, _U64, _P]),
    "haste_sgd_sr_step_f16": (ctypes.c_int, [_P, _P, _I32, _P, _I64, _F32, _F32, _F32, _I32, _I32,
                                         _U64, _U64, _P]),
    "haste_sgd_sr_step_multi": (ctypes.c_int, [ctypes.POINTER(SgdTensor), _I32, _I32, _F32, _F32,
                                               _F32, _I32, _I32, _U64, _P]),
    "haste_transpose_features": (ctypes.c_int, [_P, _I64, _P, _I64, _I64, _I64, _P]),
    "haste_rewire": (ctypes.c_int, [_P, _I32, _P, _P, _P, _I64, _I64, _I64, _I64, _I32, _F32,
                                    _I64, _I32, _I32, _F32, _U64, _P]),
    "haste_rewire_scores": (ctypes.c_int, [_P, _I32, _P, _I32, _I32, _P, _I64, _I64, _I64, _P]),
    "haste_rewire_ex": (ctypes.c_int, [_P, _I32, _P, _P, _I32, _I32, _P, _P, _P, _P, _I64, _I64,
                                       _I64, _I64, _I32, _F32, _I64, _I32, _I32, _F32, _U64,
                                       _P]),
}

_lib = None
_lock = threading.Lock()


class HasteError(RuntimeError):
    """Raised when a libhaste_ffi call returns a non-zero status."""


def lib() -> ctypes.CDLL:
    """Load (once) and return libhaste_ffi.so; raises if it is absent."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise ImportError(
                    f"haste_amd: HIP library not built ({LIB_PATH} missing); "
                    "run __graft_entry__.build() or `make -C haste_amd`")
            L = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(L, name)
                fn.restype = res
                fn.argtypes = args
            _lib = L
    return _lib


def last_error() -> str:
    msg = lib().haste_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc != HASTE_OK:
        raise HasteError(last_error() or f"libhaste_ffi error {rc}")


def call(name: str, *args) -> None:
    """Call a status-returning entry point and raise on failure."""
    check(getattr(lib(), name)(*args))
