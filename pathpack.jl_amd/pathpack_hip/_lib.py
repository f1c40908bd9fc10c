"""ctypes binding of libpathpack_hip.so (the C ABI in include/pathpack_hip.h).

The library is loaded from this package directory; there is no fallback: if it is missing, importing the binding
raises, and the solver cannot run.
"""

from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIBPATH = os.path.join(HERE, "libpathpack_hip.so")

PP_OK, PP_EINVAL, PP_ENOMEM, PP_EUNSUPPORTED, PP_EHIP, PP_ENODEV = range(6)

EXPORTS = [
    "pp_init", "pp_destroy", "pp_last_error", "pp_synchronize", "pp_stream",
    "pp_symbolic", "pp_symbolic_given", "pp_sym_size", "pp_sym_export", "pp_sym_stats", "pp_sym_destroy",
    "pp_factor", "pp_factor_device", "pp_refactor", "pp_fac_export", "pp_fac_destroy",
    "pp_star", "pp_mstar", "pp_star_sources", "pp_lmul", "pp_rmul", "pp_sgemx", "pp_getrf_star_batched",
    "pp_buffer_alloc", "pp_buffer_free", "pp_upload", "pp_download", "pp_copy", "pp_calibrate_valu", "pp_set_timing",
    "pp_get_timing", "pp_set_debug", "pp_sgetrs", "pp_sgetrs_noalloc", "pp_sym_components",
    "pp_dense_factor", "pp_dense_refactor", "pp_dense_sgetrf",
]


class PathpackError(RuntimeError):
    """A failure reported by libpathpack_hip (status code and message)."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


class PathpackArgumentError(PathpackError, ValueError):
    """Invalid argument (the reference's ArgumentError)."""


class PathpackMemoryError(PathpackError, MemoryError):
    """Not enough device memory; nothing was launched."""


class PathpackUnsupportedError(PathpackError, TypeError):
    """Unsupported semiring / element type."""


class PathpackDeviceError(PathpackError):
    """A HIP runtime failure, or no usable GPU."""


def _err(status: int, msg: str) -> PathpackError:
    cls = {PP_EINVAL: PathpackArgumentError, PP_ENOMEM: PathpackMemoryError,
           PP_EUNSUPPORTED: PathpackUnsupportedError}.get(status, PathpackDeviceError)
    return cls(status, msg)


_lib = None

c_i64 = ctypes.c_int64
c_i64p = ctypes.POINTER(ctypes.c_int64)
c_vp = ctypes.c_void_p


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIBPATH):
            raise ImportError(f"{LIBPATH} is not built (run __graft_entry__.build() or python -m pathpack_hip.build)")
        L = ctypes.CDLL(LIBPATH)
        L.pp_last_error.restype = ctypes.c_char_p
        L.pp_last_error.argtypes = [c_vp]
        for name in EXPORTS:
            if name != "pp_last_error":
                getattr(L, name).restype = ctypes.c_int
        L.pp_init.argtypes = [ctypes.POINTER(c_vp), ctypes.c_int]
        L.pp_destroy.argtypes = [c_vp]
        L.pp_synchronize.argtypes = [c_vp]
        L.pp_stream.argtypes = [c_vp, ctypes.POINTER(c_vp)]
        L.pp_symbolic.argtypes = [c_i64, c_vp, c_vp, ctypes.c_int, ctypes.c_int, c_vp, ctypes.POINTER(c_vp)]
        L.pp_symbolic_given.argtypes = [c_i64, c_vp, c_vp, c_vp, c_i64, c_vp, ctypes.POINTER(c_vp)]
        L.pp_sym_size.argtypes = [c_vp, c_i64p, c_i64p, c_i64p, c_i64p]
        L.pp_sym_export.argtypes = [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]
        L.pp_sym_stats.argtypes = [c_vp, ctypes.POINTER(ctypes.c_double)]
        L.pp_sym_destroy.argtypes = [c_vp]
        L.pp_sym_components.argtypes = [c_vp, c_i64p, c_vp, c_i64p, c_vp, c_vp, c_vp]
        L.pp_factor.argtypes = [c_vp, c_vp, ctypes.c_int, ctypes.c_int, c_vp, ctypes.POINTER(c_vp)]
        L.pp_factor_device.argtypes = [c_vp, c_vp, ctypes.c_int, ctypes.c_int, c_vp, ctypes.POINTER(c_vp)]
        L.pp_refactor.argtypes = [c_vp, c_vp, c_vp, ctypes.c_int]
        L.pp_dense_factor.argtypes = [c_vp, ctypes.c_int, ctypes.c_int, c_i64, c_vp, c_i64, ctypes.c_int,
                                      ctypes.POINTER(c_vp)]
        L.pp_dense_refactor.argtypes = [c_vp, c_vp, c_vp, c_i64, ctypes.c_int]
        L.pp_dense_sgetrf.argtypes = [c_vp, ctypes.c_int, ctypes.c_int, c_i64, c_vp, c_i64]
        L.pp_fac_export.argtypes = [c_vp, c_vp, c_vp, c_vp, c_vp, c_vp]
        L.pp_fac_destroy.argtypes = [c_vp]
        L.pp_star.argtypes = [c_vp, c_vp, c_vp, c_i64, ctypes.c_int]
        L.pp_mstar.argtypes = [c_vp, c_vp, ctypes.c_int, ctypes.c_int, c_vp, ctypes.c_int, c_vp, c_i64, ctypes.c_int,
                               ctypes.POINTER(c_vp)]
        L.pp_star_sources.argtypes = [c_vp, c_vp, ctypes.c_int, c_i64, c_vp, c_vp, c_i64, ctypes.c_int]
        L.pp_lmul.argtypes = [c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_int]
        L.pp_rmul.argtypes = [c_vp, c_vp, c_vp, c_i64, c_i64, ctypes.c_int]
        L.pp_sgemx.argtypes = [c_vp, ctypes.c_int, ctypes.c_int, c_i64, c_i64, c_i64, c_vp, c_i64, c_vp, c_i64, c_vp,
                               c_i64]
        L.pp_getrf_star_batched.argtypes = [c_vp, ctypes.c_int, ctypes.c_int, c_i64, c_i64, c_vp, c_vp, c_vp]
        L.pp_buffer_alloc.argtypes = [c_vp, ctypes.c_size_t, ctypes.POINTER(c_vp)]
        L.pp_buffer_free.argtypes = [c_vp, c_vp]
        L.pp_upload.argtypes = [c_vp, c_vp, c_vp, ctypes.c_size_t]
        L.pp_download.argtypes = [c_vp, c_vp, c_vp, ctypes.c_size_t]
        L.pp_copy.argtypes = [c_vp, c_vp, c_vp, ctypes.c_size_t]
        L.pp_calibrate_valu.argtypes = [c_vp, ctypes.c_int, c_i64, ctypes.POINTER(ctypes.c_double),
                                        ctypes.POINTER(ctypes.c_double)]
        L.pp_set_timing.argtypes = [c_vp, ctypes.c_int]
        L.pp_get_timing.argtypes = [c_vp, ctypes.POINTER(ctypes.c_double)]
        L.pp_set_debug.argtypes = [c_vp, ctypes.c_int]
        L.pp_sgetrs.argtypes = [c_vp, c_vp, ctypes.c_int, ctypes.c_int, c_vp, c_i64, c_i64, ctypes.c_int]
        L.pp_sgetrs_noalloc.argtypes = [c_vp, c_vp, ctypes.c_int, ctypes.c_int, c_vp, c_i64, c_i64]
        _lib = L
    return _lib


def check(status: int, ctx=None) -> None:
    if status != PP_OK:
        msg = lib().pp_last_error(ctx)
        raise _err(status, msg.decode() if msg else f"status {status}")
