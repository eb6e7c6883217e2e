"""ctypes binding of ``librnrqr.so`` (the C ABI declared in ``include/rnrqr.h``).

The library is built in-tree by ``build.build_library()`` (``__graft_entry__.build()``
calls it).  Loading fails loudly with :class:`NativeLibraryMissing` when it has not
been built: the package has no CPU or pure-PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import os
import threading

LIB_NAME = "librnrqr.so"
LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), LIB_NAME)

RNR_OK = 0
RNR_ERR_INVALID_ARG = 1
RNR_ERR_UNSUPPORTED_N = 2
RNR_ERR_WORKSPACE = 3
RNR_ERR_HIP = 4
RNR_ERR_MISALIGNED = 5
RNR_ERR_SCRATCH_LIMIT = 6
RNR_NOALLOC_SCRATCH_BYTES = 128 << 20
RNR_MAX_N = 2048
RNR_QR_TIMED_EVENTS = 12
# the stages of rnr_qr_f32 in order (what rnr_qr_f32_timed's events bracket)
QR_STAGES = ("lu", "gram_L", "chol_1", "wblk_1", "trsm_1", "gram_Q1", "chol_2", "wblk_2", "trsm_2", "chart",
             "closure")

_i64 = ctypes.c_int64
_vp = ctypes.c_void_p
_sz = ctypes.c_size_t
_u64 = ctypes.c_uint64
_szp = ctypes.POINTER(ctypes.c_size_t)
_int = ctypes.c_int

# name -> (restype, argtypes); mirrors include/rnrqr.h
SIGNATURES = {
    "rnr_status_string": (ctypes.c_char_p, [_int]),
    "rnr_version": (ctypes.c_char_p, []),
    "rnr_qr_f32_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_qr_f32": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "rnr_qr_f32_noalloc": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp]),
    "rnr_qr_f32_timed": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp,
                                ctypes.POINTER(ctypes.c_void_p), _int]),
    "rnr_lu_f32_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_lu_f32": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "rnr_cholqr_f32_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_cholqr_f32": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
    "rnr_frame_f32_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_frame_f32": (_int, [_vp, _i64, _i64, _i64, _vp, _vp, _vp, _sz, _vp]),
    "rnr_chart_f32": (_int, [_vp, _i64, _i64, _vp, _vp, _vp]),
    "rnr_generate_workspace": (_int, [_int, _i64, _i64, _szp]),
    "rnr_generate_f32": (_int, [_int, _i64, _i64, _u64, _vp, _vp, _sz, _vp]),
    "rnr_hh_geqrf_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_hh_geqrf_f32": (_int, [_vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "rnr_orgqr_f32_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_orgqr_f32": (_int, [_vp, _vp, _i64, _i64, _vp, _vp, _sz, _vp]),
    "rnr_ormqr_f32_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_ormqr_f32": (_int, [_vp, _vp, _i64, _i64, _vp, _i64, _i64, _i64, _int, _vp, _sz, _vp]),
    "rnr_check_f64_workspace": (_int, [_i64, _i64, _szp]),
    "rnr_check_f64": (_int, [_vp, _i64, _vp, _vp, _i64, _i64, _vp, _vp, _vp, _vp, _sz, _vp]),
}


class NativeLibraryMissing(RuntimeError):
    """librnrqr.so is not built (run ``__graft_entry__.build()``)."""


class RnrError(RuntimeError):
    """A non-zero rnr_status from the C ABI."""

    def __init__(self, fn: str, status: int, text: str):
        super().__init__(f"{fn} failed with status {status}: {text}")
        self.status = status


_lock = threading.Lock()
_lib = None


def lib() -> ctypes.CDLL:
    """The loaded library with argument types set (loaded once per process)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise NativeLibraryMissing(
                    f"{LIB_PATH} is missing; build it with __graft_entry__.build() "
                    "(this package has no CPU fallback)")
            handle = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(handle, name)
                fn.restype = res
                fn.argtypes = args
            _lib = handle
    return _lib


def status_string(status: int) -> str:
    return lib().rnr_status_string(int(status)).decode()


def check(fn: str, status: int) -> None:
    if status != RNR_OK:
        raise RnrError(fn, status, status_string(status))


def workspace_bytes(kind: str, batch: int, n: int) -> int:
    """Workspace size for one of "qr", "lu", "cholqr", "frame", "check", "hh_geqrf", "orgqr", "ormqr"."""
    out = ctypes.c_size_t(0)
    name = {"check": "rnr_check_f64_workspace", "hh_geqrf": "rnr_hh_geqrf_workspace",
            "orgqr": "rnr_orgqr_f32_workspace", "ormqr": "rnr_ormqr_f32_workspace"}.get(
        kind, f"rnr_{kind}_f32_workspace")
    check(name, getattr(lib(), name)(int(batch), int(n), ctypes.byref(out)))
    return int(out.value)
