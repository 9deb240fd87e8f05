"""ctypes binding of ``libttc_lqr.so`` (the C ABI declared in ``include/ttc_lqr.h``).

The library is built in-tree by ``ttc-net_amd/csrc/build.py`` into
``ttc-net_amd/lib/libttc_lqr.so``.  There is no fallback: if the library is
missing, importing the HIP solver raises, so a GPU run can never silently
take another code path.
"""
from __future__ import annotations

import ctypes
import os

__all__ = ["lib", "lib_path", "LIB_NAME", "TTCLQRError", "check", "FLAG_FP64_RICCATI", "FLAG_ROW_KERNEL",
           "FLAG_STABLE_BWD", "FLAG_RICCATI_STEPS", "FLAG_COMPACT_STASH", "FLAG_FP64_RESCUE", "FLAG_FP64_FALLBACK",
           "FLAG_KEEP_EXPANDED", "FLAG_RESCUE_V1", "FLAG_RESCUE_GAINS"]

FLAG_FP64_RICCATI = 1  # TTC_LQR_FLAG_FP64_RICCATI
FLAG_ROW_KERNEL = 2    # TTC_LQR_FLAG_ROW_KERNEL
FLAG_STABLE_BWD = 4    # TTC_LQR_FLAG_STABLE_BWD
FLAG_RICCATI_STEPS = 8  # TTC_LQR_FLAG_RICCATI_STEPS
FLAG_COMPACT_STASH = 16  # TTC_LQR_FLAG_COMPACT_STASH
FLAG_FP64_RESCUE = 32  # TTC_LQR_FLAG_FP64_RESCUE
FLAG_FP64_FALLBACK = 64  # TTC_LQR_FLAG_FP64_FALLBACK
FLAG_KEEP_EXPANDED = 128  # TTC_LQR_FLAG_KEEP_EXPANDED
FLAG_RESCUE_V1 = 256  # TTC_LQR_FLAG_RESCUE_V1
FLAG_RESCUE_GAINS = 512  # TTC_LQR_FLAG_RESCUE_GAINS

LIB_NAME = "libttc_lqr.so"
_HERE = os.path.dirname(os.path.abspath(__file__))
_DEFAULT = os.path.normpath(os.path.join(_HERE, "..", "..", "lib", LIB_NAME))


class TTCLQRError(RuntimeError):
    pass


def lib_path() -> str:
    return os.environ.get("TTC_LQR_LIB", _DEFAULT)


def _load():
    path = lib_path()
    if not os.path.exists(path):
        raise ImportError(
            f"{LIB_NAME} not found at {path}; build it with `python ttc-net_amd/csrc/build.py` "
            "(or __graft_entry__.build()).  The HIP solver has no non-native fallback.")
    L = ctypes.CDLL(path)
    f32p = ctypes.c_void_p
    i64, i32, sz = ctypes.c_int64, ctypes.c_int32, ctypes.c_size_t
    L.ttc_lqr_version.restype = ctypes.c_char_p
    L.ttc_lqr_version.argtypes = []
    L.ttc_lqr_strerror.restype = ctypes.c_char_p
    L.ttc_lqr_strerror.argtypes = [ctypes.c_int]
    L.ttc_lqr_supported.restype = ctypes.c_int
    L.ttc_lqr_supported.argtypes = [i32, i32]
    L.ttc_lqr_supported_flags.restype = ctypes.c_int
    L.ttc_lqr_supported_flags.argtypes = [i32, i32, i32]
    L.ttc_lqr_stash_bytes.restype = sz
    L.ttc_lqr_stash_bytes.argtypes = [i64, i32, i32, i32, i32]
    L.ttc_lqr_workspace_bytes.restype = sz
    L.ttc_lqr_workspace_bytes.argtypes = [i64, i32, i32, i32, i32, i32, i32]
    L.ttc_lqr_fallback_bytes.restype = sz
    L.ttc_lqr_fallback_bytes.argtypes = [i64, i32, i32, i32, i32]
    L.ttc_lqr_forward.restype = ctypes.c_int
    L.ttc_lqr_forward.argtypes = [f32p] * 9 + [i64, i32, i32, i32, i32, i32] + [f32p, f32p, f32p, ctypes.c_void_p]
    L.ttc_lqr_forward_workspace_bytes.restype = sz
    L.ttc_lqr_forward_workspace_bytes.argtypes = [i64, i32, i32, i32, i32, i32]
    L.ttc_lqr_forward_ws.restype = ctypes.c_int
    L.ttc_lqr_forward_ws.argtypes = ([f32p] * 9 + [i64, i32, i32, i32, i32, i32] + [f32p, f32p, ctypes.c_void_p, sz]
                                     + [f32p, ctypes.c_void_p])
    L.ttc_lqr_backward.restype = ctypes.c_int
    L.ttc_lqr_backward.argtypes = ([f32p] * 11 + [i64, i32, i32, i32, i32, i32] + [f32p] + [f32p] * 9
                                   + [ctypes.c_void_p, sz, ctypes.c_float, f32p, ctypes.POINTER(ctypes.c_int64),
                                      ctypes.c_void_p])
    L.ttc_lqr_compact_stash_bytes.restype = sz
    L.ttc_lqr_compact_stash_bytes.argtypes = [i64, i32, i32, i32]
    L.ttc_lqr_expanded_bytes.restype = sz
    L.ttc_lqr_expanded_bytes.argtypes = [i64, i32, i32, i32]
    L.ttc_lqr_rescue_stash_bytes.restype = sz
    L.ttc_lqr_rescue_stash_bytes.argtypes = [i64, i32, i32, i32]
    L.ttc_lqr_rescue_gains_bytes.restype = sz
    L.ttc_lqr_rescue_gains_bytes.argtypes = [i64, i32, i32, i32, i32]
    L.ttc_lqr_factored_workspace_bytes.restype = sz
    L.ttc_lqr_factored_workspace_bytes.argtypes = [i64, i32, i32, i32, i32, i32, i32, i32, i32, i32, i32]
    L.ttc_lqr_forward_factored.restype = ctypes.c_int
    L.ttc_lqr_forward_factored.argtypes = ([f32p] * 11 + [i64, i32, i32, i32, i32, i32, i32, i32]
                                           + [f32p, f32p, ctypes.c_void_p, sz, f32p, ctypes.c_void_p])
    L.ttc_lqr_backward_factored.restype = ctypes.c_int
    L.ttc_lqr_backward_factored.argtypes = ([f32p] * 13 + [i64, i32, i32, i32, i32, i32, i32, i32] + [f32p]
                                            + [f32p] * 11 + [ctypes.c_void_p, sz, ctypes.c_float, f32p,
                                                             ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p])
    L.ttc_lqr_rescale.restype = ctypes.c_int
    L.ttc_lqr_rescale.argtypes = [f32p, f32p, i64, i32, i32, i32, i32, f32p, ctypes.c_void_p]
    L.ttc_lqr_rescale_backward.restype = ctypes.c_int
    L.ttc_lqr_rescale_backward.argtypes = [f32p, f32p, f32p, i64, i32, i32, i32, i32, f32p, ctypes.c_void_p]
    L.ttc_lqr_noalloc_scratch_bytes.restype = sz
    L.ttc_lqr_noalloc_scratch_bytes.argtypes = []
    L.ttc_lqr_backward_noalloc.restype = ctypes.c_int
    L.ttc_lqr_backward_noalloc.argtypes = ([f32p] * 11 + [i64, i32, i32, i32, i32, i32] + [f32p] + [f32p] * 9
                                           + [ctypes.c_float, f32p, ctypes.POINTER(ctypes.c_int64), ctypes.c_void_p])
    L.ttc_lqr_forward_host.restype = ctypes.c_int
    L.ttc_lqr_forward_host.argtypes = [f32p] * 9 + [i64, i32, i32, i32, i32] + [f32p, f32p, i32]
    L.ttc_lqr_backward_host.restype = ctypes.c_int
    L.ttc_lqr_backward_host.argtypes = ([f32p] * 10 + [i64, i32, i32, i32, i32] + [f32p] * 9
                                        + [ctypes.c_float, f32p, i32])
    for suffix in ("", "_bf16"):
        getattr(L, "ttc_lqr_forward_factored" + suffix).restype = ctypes.c_int
        getattr(L, "ttc_lqr_forward_factored" + suffix).argtypes = L.ttc_lqr_forward_factored.argtypes
        getattr(L, "ttc_lqr_backward_factored" + suffix).restype = ctypes.c_int
        getattr(L, "ttc_lqr_backward_factored" + suffix).argtypes = L.ttc_lqr_backward_factored.argtypes
    return L


lib = _load()


def check(rc: int, what: str) -> None:
    if rc != 0:
        raise TTCLQRError(f"{what} failed: {lib.ttc_lqr_strerror(rc).decode()} (code {rc})")
