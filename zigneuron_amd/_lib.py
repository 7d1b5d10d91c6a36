"""ctypes binding of libzn_hip.so (the C ABI in include/zn_hip.h).

The library and its gfx950 code objects live in ``zigneuron_amd/lib/`` and are
built by ``__graft_entry__.build()`` (``make -C zigneuron_amd/csrc``).  There
is no fallback: if the library is missing, loading raises.
"""
from __future__ import annotations

import ctypes
import os

PKG_DIR = os.path.dirname(os.path.abspath(__file__))
LIB_DIR = os.path.join(PKG_DIR, "lib")
LIB_PATH = os.path.join(LIB_DIR, "libzn_hip.so")

# Status codes (include/zn_hip.h)
ZN_OK = 0
ZN_ERR_NO_DEVICE = -1
ZN_ERR_CODE_OBJECT = -2
ZN_ERR_SYMBOL = -3
ZN_ERR_INVALID_ARG = -4
ZN_ERR_OOM = -5
ZN_ERR_LAUNCH = -6
ZN_ERR_HIP = -7
ZN_ERR_OVERFLOW = -8

LAYOUT_NN, LAYOUT_NT, LAYOUT_TN = 0, 1, 2
TILE_AUTO = -1
TILES = {"auto": -1, "256x128": 0, "128x128": 1, "128x64": 2, "64x64": 3, "32x32": 4, "128x128k32": 5, "64x64k16": 6,
         "256x256": 7}
ACT_LINEAR, ACT_RELU, ACT_SIGMOID, ACT_TANH = 0, 1, 2, 3


class ZnError(RuntimeError):
    """A non-zero status from the C ABI (the Zig error-union analogue)."""

    def __init__(self, status: int, where: str, message: str):
        super().__init__(f"{where}: {message}")
        self.status = status


class NoDeviceError(ZnError):
    pass


class CodeObjectError(ZnError):
    pass


class SymbolError(ZnError):
    pass


class InvalidArgumentError(ZnError, ValueError):
    pass


class OutOfMemoryError(ZnError, MemoryError):
    pass


class LaunchError(ZnError):
    pass


class HipError(ZnError):
    pass


class OverflowError_(ZnError, OverflowError):
    pass


_ERRORS = {
    ZN_ERR_NO_DEVICE: NoDeviceError,
    ZN_ERR_CODE_OBJECT: CodeObjectError,
    ZN_ERR_SYMBOL: SymbolError,
    ZN_ERR_INVALID_ARG: InvalidArgumentError,
    ZN_ERR_OOM: OutOfMemoryError,
    ZN_ERR_LAUNCH: LaunchError,
    ZN_ERR_HIP: HipError,
    ZN_ERR_OVERFLOW: OverflowError_,
}

P = ctypes.c_void_p
S = ctypes.c_size_t
I = ctypes.c_int
I64 = ctypes.c_int64
F = ctypes.c_float


class DeviceInfo(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char * 64), ("compute_units", ctypes.c_int32),
                ("clock_khz", ctypes.c_int32), ("total_mem", ctypes.c_int64)]


# name -> (restype, argtypes); must match include/zn_hip.h exactly.
SIGNATURES = {
    "zn_hip_abi_version": (I, []),
    "zn_hip_available": (I, []),
    "zn_hip_create": (I, [I, ctypes.c_char_p, ctypes.POINTER(P)]),
    "zn_hip_destroy": (I, [P]),
    "zn_hip_status_string": (ctypes.c_char_p, [I]),
    "zn_hip_last_hip_error": (I, [P]),
    "zn_hip_device_info": (I, [P, ctypes.POINTER(DeviceInfo)]),
    "zn_hip_stream": (P, [P]),
    "zn_hip_alloc": (I, [P, S, ctypes.POINTER(P)]),
    "zn_hip_free": (I, [P, P]),
    "zn_hip_h2d": (I, [P, P, P, S]),
    "zn_hip_d2h": (I, [P, P, P, S]),
    "zn_hip_h2d_async": (I, [P, P, P, S]),
    "zn_hip_d2h_async": (I, [P, P, P, S]),
    "zn_hip_fill_f32": (I, [P, P, F, I64]),
    "zn_hip_copy_f32": (I, [P, P, P, I64]),
    "zn_hip_hold_stream": (I, [P, F]),
    "zn_hip_sync": (I, [P]),
    "zn_hip_graph_begin": (I, [P]),
    "zn_hip_graph_end": (I, [P, ctypes.POINTER(P)]),
    "zn_hip_graph_launch": (I, [P, P]),
    "zn_hip_graph_destroy": (I, [P]),
    "zn_hip_event_create": (I, [P, ctypes.POINTER(P)]),
    "zn_hip_event_record": (I, [P, P]),
    "zn_hip_event_elapsed_ms": (I, [P, P, ctypes.POINTER(F)]),
    "zn_hip_event_destroy": (I, [P]),
    "zn_hip_set_gemm_tile": (I, [P, I]),
    "zn_hip_set_gemm_splits": (I, [P, I]),
    "zn_hip_set_gemm_persistent": (I, [P, I]),
    "zn_hip_set_gemm_wave_split": (I, [P, I]),
    "zn_hip_sgemm": (I, [P, I, I64, I64, I64, P, I64, P, I64, P, I64, I, P, I]),
    "zn_hip_sgemm_noalloc": (I, [P, I, I64, I64, I64, P, I64, P, I64, P, I64, I, P, I]),
    "zn_hip_sgemm_strided_batched": (I, [P, I, I64, I64, I64, P, I64, I64, P, I64, I64, P, I64, I64, I64, I, P, I]),
    "zn_hip_add_bias": (I, [P, P, P, I64, I64]),
    "zn_hip_activation_forward": (I, [P, I, P, P, I64]),
    "zn_hip_activation_backward": (I, [P, I, P, P, P, I64]),
    "zn_hip_accumulate_bias": (I, [P, P, P, I64, I64]),
    "zn_hip_mat_mul": (I, [P, P, S, P, S, P, S, S, S, S, I]),
    "zn_hip_mat_mul_batch": (I, [P, P, S, P, S, P, S, S, S, S, I]),
    "zn_hip_mat_mul_transpose_a": (I, [P, P, S, P, S, P, S, S, S, S, I]),
    "zn_hip_mat_mul_transpose_b": (I, [P, P, S, P, S, P, S, S, S, S, I]),
    "zn_hip_mat_mul_bias": (I, [P, P, S, P, S, P, S, P, S, S, S, S]),
    "zn_hip_mat_mul_bias_relu": (I, [P, P, S, P, S, P, S, P, S, S, S, S]),
    "zn_hip_mat_mul_bias_sigmoid": (I, [P, P, S, P, S, P, S, P, S, S, S, S]),
    "zn_hip_mat_mul_bias_tanh": (I, [P, P, S, P, S, P, S, P, S, S, S, S]),
    "zn_hip_add_bias_host": (I, [P, P, S, P, S]),
    "zn_hip_activation_forward_host": (I, [P, I, P, S, P, S]),
    "zn_hip_activation_backward_host": (I, [P, I, P, S, P, S, P, S]),
    "zn_hip_accumulate_bias_host": (I, [P, P, S, P, S]),
    "zn_hip_dense_backward": (I, [P, I] + [P] * 8 + [I64] * 3),
    "zn_hip_dense_backward_chain": (I, [P, I] + [P] * 8 + [I64] * 3 + [I, I, P, P]),
    "zn_hip_dense_pair_forward": (I, [P, I, P, P, P, P, I, P, P, P] + [I64] * 4),
    "zn_hip_dense_pair_backward": (I, [P, I] + [P] * 7 + [I] + [P] * 7 + [I64] * 4),
    "zn_hip_im2col": (I, [P, P, P] + [I64] * 12),
    "zn_hip_conv2d_forward_im2col": (I, [P, P, P, P, P] + [I64] * 13),
    "zn_hip_conv2d_forward_direct": (I, [P, P, P, P, P] + [I64] * 13),
    "zn_hip_col2im": (I, [P, P, P] + [I64] * 12),
    "zn_hip_conv2d_backward_im2col": (I, [P] + [P] * 6 + [I64] * 13),
    "zn_hip_conv2d_backward_direct": (I, [P] + [P] * 6 + [I64] * 13),
    "zn_hip_softmax_rows": (I, [P, P, P, I64, I64, F]),
    "zn_hip_attention_forward": (I, [P, P, P, P, P, I64, I64, I64, F]),
    "zn_hip_conv2d_forward_host": (I, [P, P, S, P, S, P, S, P, S] + [S] * 11),
    "zn_hip_conv2d_backward_host": (I, [P, P, S, P, S, P, S, P, S, P, S, P, S] + [S] * 12),
    "zn_hip_attention_forward_host": (I, [P, P, S, P, S, P, S, P, S, P, S, S, S, F]),
}

_lib = None


def load() -> ctypes.CDLL:
    """Load libzn_hip.so once; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise CodeObjectError(ZN_ERR_CODE_OBJECT, "zigneuron_amd",
                                  f"{LIB_PATH} is missing; run __graft_entry__.build()")
        lib = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        _lib = lib
    return _lib


def status_string(status: int) -> str:
    return load().zn_hip_status_string(status).decode()


def check(status: int, where: str) -> None:
    if status != ZN_OK:
        cls = _ERRORS.get(status, ZnError)
        raise cls(status, where, status_string(status))
