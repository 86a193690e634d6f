"""Loader for libgomlx_hip.so, the C ABI declared in include/gomlx_hip.h.

The library is the product: every op in this package runs through it.  There is
no CPU fallback — if the library is missing the import fails loudly.
"""
from __future__ import annotations

import ctypes
import os

_PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
# GHIP_LIB_PATH selects another build of the same ABI (e.g. the sanitizer build
# of the host code, `make -C go-darwinml_amd/csrc asan`).
LIB_PATH = os.environ.get("GHIP_LIB_PATH") or os.path.join(_PKG_ROOT, "lib", "libgomlx_hip.so")
CSRC_DIR = os.path.join(_PKG_ROOT, "csrc")

# Dtype numbering of include/gomlx_hip.h (the reference's MPSGraphDType).
DT_BOOL, DT_INT8, DT_INT16, DT_INT32, DT_INT64 = 0, 1, 2, 3, 4
DT_FLOAT16, DT_BFLOAT16, DT_FLOAT32, DT_FLOAT64 = 5, 6, 7, 8
DT_UINT8, DT_UINT16, DT_UINT32, DT_UINT64 = 9, 10, 11, 12


class GHipError(ctypes.Structure):
    _fields_ = [("code", ctypes.c_int), ("message", ctypes.c_char_p)]


class BackendError(RuntimeError):
    """Raised when a C entry point returns a non-zero GHIP_ERR_* code."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[code {code}] {message}")
        self.code = code


_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p
_f32 = ctypes.c_float
_errp = ctypes.POINTER(GHipError)

# name -> argtypes (every entry point returns int except where noted).
SIGNATURES = {
    "ghip_softmax_rows": [_int, _vp, _vp, _i64, _i64, _int, _vp, _errp],
    "ghip_scale_mask_softmax_rows": [_int, _vp, _vp, _i64, _i64, _i64, _f32, _int, _vp, _vp, _errp],
    "ghip_rmsnorm_rows": [_int, _vp, _vp, _vp, _i64, _i64, _f32, _vp, _errp],
    "ghip_layernorm_rows": [_int, _vp, _vp, _vp, _vp, _i64, _i64, _f32, _vp, _errp],
    "ghip_gemm_batched": [_int, _int, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
                          _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _errp],
    "ghip_gemm_grouped": [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _i64, ctypes.POINTER(_vp), _i64, _i64,
                          ctypes.POINTER(_vp), _i64, _vp, _errp],
    "ghip_gemm_batched_ws": [_int, _int, _i64, _i64, _i64, _i64, _vp, _i64, _i64, _i64,
                             _vp, _i64, _i64, _i64, _vp, _i64, _i64, _i64, _vp, _i64, _vp, _errp],
    "ghip_gemm_grouped_ws": [_int, _int, _int, _i64, _i64, _i64, _vp, _i64, _i64, ctypes.POINTER(_vp), _i64,
                             _i64, ctypes.POINTER(_vp), _i64, _vp, _i64, _vp, _errp],
    "ghip_gather_rows": [_vp, _i64, _i64, _vp, _i64, _vp, _vp, _errp],
    "ghip_argminmax": [_int, _vp, _i64, _i64, _i64, _int, _int, _vp, _vp, _errp],
    "ghip_iota": [_int, _vp, _i64, _i64, _i64, _vp, _errp],
    "ghip_device_name": [_int, ctypes.c_char_p, ctypes.c_size_t, _errp],
    "ghip_sdpa_fwd": [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                      ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                      ctypes.POINTER(_i64), _f32, _int, _vp, _errp],
    "ghip_sdpa_fwd_masked": [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                             ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                             ctypes.POINTER(_i64), _vp, _int, ctypes.POINTER(_i64), _f32, _int, _vp,
                             _errp],
    "ghip_sdpa_fwd_masked_ws": [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                ctypes.POINTER(_i64), ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                                ctypes.POINTER(_i64), _vp, _int, ctypes.POINTER(_i64), _f32, _int, _vp, _i64,
                                _vp, _errp],
    "ghip_scale_mask_softmax_rows_ex": [_int, _vp, _vp, _i64, _i64, _i64, _i64, _f32, _int, _vp, _int,
                                        ctypes.POINTER(_i64), _vp, _errp],
    "ghip_copy_strided": [_int, _vp, _vp, _int, ctypes.POINTER(_i64), ctypes.POINTER(_i64),
                          ctypes.POINTER(_i64), _vp, _errp],
    "ghip_softmax_cols": [_int, _vp, _vp, _i64, _i64, _i64, _int, _vp, _errp],
    "ghip_layernorm_cols": [_int, _vp, _vp, _vp, _vp, _i64, _i64, _i64, _f32, _vp, _errp],
}

# name -> argtypes of the entry points that return int64_t.
SIGNATURES_I64 = {
    "ghip_sdpa_workspace_bytes": [_int, _i64, _i64, _i64, _i64, _i64, _i64, _int],
    "ghip_gemm_workspace_bytes": [_int, _int, _i64, _i64, _i64, _i64],
}

_lib = None


def load():
    """Returns the loaded library (raises if it was never built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise ImportError(
            f"gomlx_hip: {LIB_PATH} is missing; build it with "
            f"`make -C {CSRC_DIR}` (or __graft_entry__.build())")
    L = ctypes.CDLL(LIB_PATH)
    for name, argtypes in SIGNATURES.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int
    for name, argtypes in SIGNATURES_I64.items():
        fn = getattr(L, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_int64
    L.ghip_version.argtypes = []
    L.ghip_version.restype = ctypes.c_char_p
    L.ghip_error_clear.argtypes = [_errp]
    L.ghip_error_clear.restype = None
    _lib = L
    return L


def call(name: str, *args) -> None:
    """Calls entry point `name` with a fresh GHipError; raises BackendError on failure."""
    L = load()
    err = GHipError(0, None)
    rc = getattr(L, name)(*args, ctypes.byref(err))
    if rc != 0:
        msg = err.message.decode() if err.message else "(no message)"
        L.ghip_error_clear(ctypes.byref(err))
        raise BackendError(rc, msg)
