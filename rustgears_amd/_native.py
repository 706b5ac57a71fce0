"""ctypes binding of librgnpu.so (include/rgnpu.h).

The library is built in-tree by rustgears_amd/build.py.  Loading fails loudly
when it is missing: there is no CPU fallback for the execution provider.
"""
from __future__ import annotations

import ctypes
import os

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "librgnpu.so")

# status codes (include/rgnpu.h)
OK = 0
ERR_INVALID = 1
ERR_SHAPE = 2
ERR_DEVICE = 3
ERR_UNSUPPORTED = 4
ERR_IO = 5
ERR_FORMAT = 6
ERR_CAPACITY = 7

# layer kinds / activation codes / precisions / capture taps
LAYER_LINEAR, LAYER_CONV2D, LAYER_CHANNEL_AFFINE = 1, 2, 3
LAYER_MAXPOOL2D, LAYER_FLATTEN, LAYER_ACTIVATION, LAYER_SOFTMAX = 4, 5, 6, 7
PRECISION_INT8, PRECISION_FP16, PRECISION_FP32 = 0, 1, 2
CAP_QACT, CAP_SCALE, CAP_ACC, CAP_OUT = 0, 1, 2, 3
CAPTURE_OFF, CAPTURE_FULL, CAPTURE_PRODUCTION = 0, 1, 2

f32p = ctypes.POINTER(ctypes.c_float)
i64p = ctypes.POINTER(ctypes.c_int64)
i32p = ctypes.POINTER(ctypes.c_int32)


class CLayer(ctypes.Structure):
    """rgnpu_layer."""

    _fields_ = [
        ("kind", ctypes.c_int32),
        ("act", ctypes.c_int32), ("act_param", ctypes.c_float),
        ("in_features", ctypes.c_int64), ("out_features", ctypes.c_int64),
        ("in_channels", ctypes.c_int64), ("out_channels", ctypes.c_int64),
        ("kernel", ctypes.c_int64), ("stride", ctypes.c_int64), ("padding", ctypes.c_int64),
        ("pool_kernel", ctypes.c_int64), ("pool_stride", ctypes.c_int64),
        ("weight", f32p), ("weight_len", ctypes.c_int64),
        ("bias", f32p), ("bias_len", ctypes.c_int64),
        ("scale", f32p), ("scale_len", ctypes.c_int64),
        ("shift", f32p), ("shift_len", ctypes.c_int64),
    ]


class COpRecord(ctypes.Structure):
    """rgnpu_op_record."""

    _fields_ = [("op", ctypes.c_char * 96), ("macs", ctypes.c_uint64), ("ns", ctypes.c_uint64),
                ("kernel_ns", ctypes.c_uint64)]


class CProfile(ctypes.Structure):
    """rgnpu_profile."""

    _fields_ = [
        ("precision", ctypes.c_int32), ("original_layers", ctypes.c_int32),
        ("fused_ops", ctypes.c_int32), ("n_records", ctypes.c_int32),
        ("fp32_weight_bytes", ctypes.c_uint64), ("npu_weight_bytes", ctypes.c_uint64),
        ("total_macs", ctypes.c_uint64), ("total_ns", ctypes.c_uint64),
    ]


# (name, restype, argtypes) for every symbol declared in include/rgnpu.h
SIGNATURES = [
    ("rgnpu_program_create", ctypes.c_int, [ctypes.POINTER(CLayer), ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                            ctypes.POINTER(ctypes.c_void_p)]),
    ("rgnpu_program_run", ctypes.c_int, [ctypes.c_void_p, f32p, i64p, ctypes.c_int32, f32p, ctypes.c_int64, i64p,
                                         i32p]),
    ("rgnpu_program_run_device", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, i64p, ctypes.c_int32,
                                                ctypes.c_void_p, ctypes.c_int64, i64p, i32p]),
    ("rgnpu_program_synchronize", ctypes.c_int, [ctypes.c_void_p]),
    ("rgnpu_program_run_device_noalloc", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, i64p, ctypes.c_int32,
                                                        ctypes.c_void_p, ctypes.c_int64, i64p, i32p]),
    ("rgnpu_program_benchmark", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, i64p, ctypes.c_int32,
                                               ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_int32,
                                               ctypes.POINTER(ctypes.c_double), ctypes.c_void_p, ctypes.c_int32]),
    ("rgnpu_program_set_profiling", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    ("rgnpu_program_profile", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(CProfile), ctypes.POINTER(COpRecord),
                                             ctypes.c_int32]),
    ("rgnpu_program_summary", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_int64]),
    ("rgnpu_program_num_ops", ctypes.c_int64, [ctypes.c_void_p]),
    ("rgnpu_program_op_label", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_char_p, ctypes.c_int64]),
    ("rgnpu_program_op_weight", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                                 f32p]),
    ("rgnpu_program_set_capture", ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
    ("rgnpu_program_capture", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int32, ctypes.c_void_p,
                                               ctypes.c_int64]),
    ("rgnpu_program_destroy", None, [ctypes.c_void_p]),
    ("rgnpu_last_error", ctypes.c_char_p, []),
    ("rgnpu_rtim_load", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ctypes.c_void_p),
                                       ctypes.POINTER(ctypes.POINTER(CLayer)), i64p]),
    ("rgnpu_rtim_free", None, [ctypes.c_void_p]),
    ("rgnpu_rtim_save", ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(CLayer), ctypes.c_int64]),
    ("rgnpu_manual_seed", None, [ctypes.c_uint64]),
    ("rgnpu_fill_uniform", None, [f32p, ctypes.c_int64]),
    ("rgnpu_fill_uniform_range", None, [f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_float]),
    ("rgnpu_fill_normal", None, [f32p, ctypes.c_int64]),
    ("rgnpu_probe_mfma_rate", ctypes.c_int, [ctypes.c_int32, ctypes.c_int64, ctypes.c_int32,
                                             ctypes.POINTER(ctypes.c_double), ctypes.POINTER(ctypes.c_double)]),
    ("rgnpu_probe_barrier_poll", ctypes.c_int, [ctypes.c_int32, ctypes.c_int32, ctypes.c_int32,
                                                ctypes.POINTER(ctypes.c_double)]),
    ("rgnpu_program_barrier_stats", ctypes.c_int, [ctypes.c_void_p, ctypes.POINTER(ctypes.c_uint64),
                                                   ctypes.POINTER(ctypes.c_uint64), ctypes.POINTER(ctypes.c_uint64)]),
    ("rgnpu_device_count", ctypes.c_int, [i32p]),
    ("rgnpu_device_alloc", ctypes.c_int, [ctypes.c_int32, ctypes.c_int64, ctypes.POINTER(ctypes.c_void_p)]),
    ("rgnpu_device_free", ctypes.c_int, [ctypes.c_void_p]),
    ("rgnpu_memcpy_h2d", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    ("rgnpu_memcpy_d2h", ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_int64]),
    ("rgnpu_device_synchronize", ctypes.c_int, []),
]

_lib = None


class RgnpuError(RuntimeError):
    """A nonzero status from librgnpu, with rgnpu_last_error()'s message."""

    def __init__(self, code: int, message: str):
        super().__init__(f"[rgnpu status {code}] {message}")
        self.code = code


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise ImportError(
                f"{LIB_PATH} is missing: build the HIP extension first "
                "(python -m rustgears_amd.build or __graft_entry__.build())")
        handle = ctypes.CDLL(LIB_PATH)
        for name, res, args in SIGNATURES:
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        _lib = handle
    return _lib


def check(status: int) -> None:
    if status != OK:
        msg = lib().rgnpu_last_error()
        raise RgnpuError(status, msg.decode() if msg else "")


def device_count() -> int:
    n = ctypes.c_int32(0)
    st = lib().rgnpu_device_count(ctypes.byref(n))
    return n.value if st == OK else 0
