"""ctypes binding of libhipbackend.so (include/laya_hip.h).

The symbol table mirrors the shape of backend-mlx's hand-written FFI
(packages/backend-mlx/src/ffi.ts:31-114): every C function is declared once
with its argument types, and `call` turns a nonzero return code into a
Python exception carrying hb_last_error() -- a failed native call never
exits the process (ffi.ts:15-16,190-201).
"""
from __future__ import annotations

import ctypes as C

from .lib import resolve_lib

U = C.c_uint64     # uintptr_t
I64 = C.c_int64
I = C.c_int
F = C.c_float
D = C.c_double
P = C.c_void_p
PI64 = C.POINTER(C.c_int64)
PU64 = C.POINTER(C.c_uint64)

# dtype codes (laya_hip.h)
HB_F32, HB_F16, HB_BF16, HB_I32, HB_BOOL, HB_U8, HB_I8, HB_U16, HB_I16, HB_U32 = range(10)
HB_EPI_BIAS, HB_EPI_RESID, HB_EPI_GEGLU = 1, 2, 4
HB_X_PANEL, HB_Y_PANEL = 8, 16  # panel-order x / y (laya_hip.h)
(HB_UN_COPY, HB_UN_SCALE, HB_UN_EXP, HB_UN_LOG, HB_UN_RELU, HB_UN_GELU, HB_UN_NEG, HB_UN_ABS, HB_UN_SQRT,
 HB_UN_RSQRT, HB_UN_TANH, HB_UN_SIGMOID, HB_UN_ERF, HB_UN_NOT) = range(14)
(HB_BIN_ADD, HB_BIN_SUB, HB_BIN_MUL, HB_BIN_DIV, HB_BIN_MAX, HB_BIN_MIN, HB_BIN_POW, HB_BIN_EQ, HB_BIN_NE,
 HB_BIN_LT, HB_BIN_LE, HB_BIN_GT, HB_BIN_GE, HB_BIN_AND, HB_BIN_OR) = range(15)
HB_RED_SUM, HB_RED_MAX, HB_RED_MIN, HB_RED_MEAN, HB_RED_ARGMAX, HB_RED_ARGMIN = range(6)
HB_SCAN_SOFTMAX, HB_SCAN_CUMSUM, HB_SCAN_SORT = range(3)

# name -> (restype, argtypes); every entry point of include/laya_hip.h
SYMBOLS: dict[str, tuple] = {
    "hb_last_error": (C.c_char_p, []),
    "hb_abi_version": (I, []),
    "hb_init": (I, [I, PU64]),
    "hb_destroy": (I, [U]),
    "hb_device_info": (I, [U, C.c_char_p, C.c_size_t]),
    "hb_alloc": (I, [U, C.c_size_t, PU64]),
    "hb_free": (I, [U, U]),
    "hb_pool_stats": (I, [U, PU64, PU64, PU64]),
    "hb_pool_trim": (I, [U]),
    "hb_upload": (I, [U, U, P, C.c_size_t]),
    "hb_download": (I, [U, P, U, C.c_size_t]),
    "hb_copy": (I, [U, U, U, C.c_size_t]),
    "hb_fill": (I, [U, U, I, C.c_size_t]),
    "hb_sync": (I, [U]),
    "hb_event_create": (I, [U, PU64]),
    "hb_event_record": (I, [U, U]),
    "hb_event_elapsed": (I, [U, U, C.POINTER(F)]),
    "hb_event_destroy": (I, [U]),
    "hb_capture_begin": (I, [U]),
    "hb_capture_end": (I, [U, PU64]),
    "hb_graph_launch": (I, [U, U]),
    "hb_graph_destroy": (I, [U, U]),
    "hb_linear": (I, [U, I, U, I64, U, U, U, I64, U, I64, I64, I64, I64, C.c_uint]),
    "hb_linear_qkv": (I, [U, I, U, I64, U, U, U, I64, I64, I64, I64, D, C.c_uint]),
    "hb_qlinear": (I, [U, I, U, I64, U, U, U, U, U, I64, U, I64, I64, I64, I64, I, I, I, C.c_uint]),
    "hb_qgather": (I, [U, U, U, U, I64, I64, I, I, I, U, I64, I, U]),
    "hb_layernorm": (I, [U, I, U, I64, I, U, U, I, U, I64, I64, F]),
    "hb_layernorm_panel": (I, [U, I, U, I64, I, U, U, U, I64, I64, F]),
    "hb_panel_pack": (I, [U, U, I64, U, I64, I64]),
    "hb_panel_unpack": (I, [U, U, U, I64, I64, I64]),
    "hb_rope": (I, [U, I, U, PI64, I, U, I64, I64, I64, I64, D]),
    "hb_sdpa": (I, [U, I, U, PI64, U, PI64, U, PI64, U, PI64, U, U, PI64, I64, I64, I64, I64, I64, F, D, D]),
    "hb_sdpa_panel": (I, [U, I, U, PI64, U, PI64, U, PI64, U, PI64, U, U, I64, I64, I64, I64, I64, F, D, D]),
    "hb_sdpa_noalloc": (I, [U, I, U, PI64, U, PI64, U, PI64, U, PI64, U, PI64, I64, I64, I64, I64, I64, F]),
    "hb_sdpa_mask_info_bytes": (I, [I64, I64, I64, C.POINTER(C.c_size_t)]),
    "hb_sdpa_mask_info": (I, [U, U, PI64, I64, I64, I64, U]),
    "hb_geglu": (I, [U, I, U, I64, I, U, I64, I64]),
    "hb_unary": (I, [U, I, I, U, PI64, I, U, PI64, PI64, I, D]),
    "hb_binary": (I, [U, I, I, U, PI64, I, U, PI64, I, U, PI64, I]),
    "hb_where": (I, [U, U, PI64, I, U, PI64, I, U, PI64, I, U, PI64, I]),
    "hb_gather": (I, [U, I, U, I64, I64, U, I64, I64, I, U]),
    "hb_reduce": (I, [U, I, I, U, I64, I64, I64, I, U]),
    "hb_scan": (I, [U, I, I, U, I64, I64, I64, I, U]),
    "hb_meanpool": (I, [U, I, U, U, I64, I64, I64, U]),
}


class HipError(RuntimeError):
    """A failed libhipbackend call; the message is hb_last_error()."""


class Native:
    """The loaded library with typed entry points."""

    def __init__(self, path: str | None = None):
        self.path = resolve_lib(path)
        self.lib = C.CDLL(self.path)
        for name, (res, args) in SYMBOLS.items():
            fn = getattr(self.lib, name)
            fn.restype = res
            fn.argtypes = args
        if self.lib.hb_abi_version() != 1:
            raise HipError(f"{self.path}: ABI version {self.lib.hb_abi_version()}, expected 1")

    def last_error(self) -> str:
        m = self.lib.hb_last_error()
        return m.decode() if m else ""

    def call(self, op: str, name: str, *args) -> None:
        rc = getattr(self.lib, name)(*args)
        if rc != 0:
            raise HipError(f"{op}: {self.last_error()}")


def i64s(vals) -> C.Array:
    """A C int64 array (strides / shapes) from a Python sequence."""
    vals = list(vals)
    return (C.c_int64 * max(1, len(vals)))(*vals)


_native: Native | None = None


def native(path: str | None = None) -> Native:
    global _native
    if _native is None or (path and path != _native.path):
        _native = Native(path)
    return _native
