"""Python access to the CPU oracle (oracle/rgref.c).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, never by the product package.  The oracle is a
plain-C restatement of the reference's NPU INT8 path (see rgref.h for the
file:line map and the list of checks that pin it).
"""
from __future__ import annotations

import ctypes
import os
import subprocess
from typing import List, Sequence

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "_build", "librgref.so")

f32p = ctypes.POINTER(ctypes.c_float)
i8p = ctypes.POINTER(ctypes.c_int8)
i32p = ctypes.POINTER(ctypes.c_int32)
i64p = ctypes.POINTER(ctypes.c_int64)

CAP_QACT, CAP_SCALE, CAP_ACC, CAP_OUT = 0, 1, 2, 3


class RefLayer(ctypes.Structure):
    _fields_ = [
        ("kind", ctypes.c_int32),
        ("in_features", ctypes.c_int32), ("out_features", ctypes.c_int32),
        ("in_channels", ctypes.c_int32), ("out_channels", ctypes.c_int32),
        ("kernel", ctypes.c_int32), ("stride", ctypes.c_int32), ("padding", ctypes.c_int32),
        ("pool_kernel", ctypes.c_int32), ("pool_stride", ctypes.c_int32),
        ("act", ctypes.c_int32), ("act_param", ctypes.c_float),
        ("weight", f32p), ("weight_len", ctypes.c_int64),
        ("bias", f32p), ("bias_len", ctypes.c_int64),
        ("scale", f32p), ("shift", f32p), ("affine_len", ctypes.c_int64),
    ]


class RefRng(ctypes.Structure):
    _fields_ = [("state", ctypes.c_uint64)]


_lib = None


def build() -> str:
    res = subprocess.run(["make", "-C", HERE], capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")
    return LIB_PATH


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        sig = [
            ("rgref_rng_new", None, [ctypes.POINTER(RefRng), ctypes.c_uint64]),
            ("rgref_rng_next_u64", ctypes.c_uint64, [ctypes.POINTER(RefRng)]),
            ("rgref_rng_uniform", ctypes.c_float, [ctypes.POINTER(RefRng)]),
            ("rgref_rng_uniform_range", ctypes.c_float, [ctypes.POINTER(RefRng), ctypes.c_float, ctypes.c_float]),
            ("rgref_rng_normal", ctypes.c_float, [ctypes.POINTER(RefRng)]),
            ("rgref_manual_seed", None, [ctypes.c_uint64]),
            ("rgref_fill_uniform", None, [f32p, ctypes.c_int64]),
            ("rgref_fill_uniform_range", None, [f32p, ctypes.c_int64, ctypes.c_float, ctypes.c_float]),
            ("rgref_fill_normal", None, [f32p, ctypes.c_int64]),
            ("rgref_act_apply", ctypes.c_float, [ctypes.c_int, ctypes.c_float, ctypes.c_float]),
            ("rgref_act_apply_array", None, [ctypes.c_int, ctypes.c_float, f32p, f32p, ctypes.c_int64]),
            ("rgref_quantize", ctypes.c_float, [f32p, ctypes.c_int64, i8p]),
            ("rgref_dot_i8", ctypes.c_int32, [i8p, i8p, ctypes.c_int64]),
            ("rgref_int8_gemm_fused", None, [i8p, ctypes.c_float, i8p, ctypes.c_float, ctypes.c_int64,
                                             ctypes.c_int64, ctypes.c_int64, f32p, ctypes.c_int, ctypes.c_float,
                                             f32p, i32p, ctypes.c_int]),
            ("rgref_out_size", ctypes.c_int64, [ctypes.c_int64] * 4),
            ("rgref_im2col", None, [f32p] + [ctypes.c_int64] * 8 + [f32p]),
            ("rgref_transpose2d", None, [f32p, ctypes.c_int64, ctypes.c_int64, f32p]),
            ("rgref_max_pool2d", None, [f32p] + [ctypes.c_int64] * 6 + [f32p, ctypes.c_int]),
            ("rgref_softmax_rows", None, [f32p, ctypes.c_int64, ctypes.c_int64, f32p]),
            ("rgref_compile", ctypes.c_void_p, [ctypes.POINTER(RefLayer), ctypes.c_int64]),
            ("rgref_compile_precision", ctypes.c_void_p, [ctypes.POINTER(RefLayer), ctypes.c_int64, ctypes.c_int]),
            ("rgref_round_fp16", ctypes.c_float, [ctypes.c_float]),
            ("rgref_matmul_f32", None, [f32p, f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, f32p, ctypes.c_int]),
            ("rgref_round_fp16_array", None, [f32p, f32p, ctypes.c_int64]),
            ("rgref_program_op_weight_fp16", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(f32p),
                                                              i64p]),
            ("rgref_fp16_gemm_fused", None, [f32p, f32p, ctypes.c_int64, ctypes.c_int64, ctypes.c_int64, f32p,
                                             ctypes.c_int, ctypes.c_float, f32p, ctypes.c_int]),
            ("rgref_program_free", None, [ctypes.c_void_p]),
            ("rgref_program_num_ops", ctypes.c_int64, [ctypes.c_void_p]),
            ("rgref_program_fp32_bytes", ctypes.c_int64, [ctypes.c_void_p]),
            ("rgref_program_npu_bytes", ctypes.c_int64, [ctypes.c_void_p]),
            ("rgref_program_original_layers", ctypes.c_int64, [ctypes.c_void_p]),
            ("rgref_program_op_label", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_char_p,
                                                        ctypes.c_int64]),
            ("rgref_program_op_weight", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64, ctypes.POINTER(i8p),
                                                         f32p, ctypes.POINTER(f32p)]),
            ("rgref_program_set_capture", None, [ctypes.c_void_p, ctypes.c_int]),
            ("rgref_program_capture", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64, ctypes.c_int,
                                                       ctypes.POINTER(ctypes.c_void_p)]),
            ("rgref_execute", ctypes.c_int, [ctypes.c_void_p, f32p, i64p, ctypes.c_int, ctypes.c_int]),
            ("rgref_program_output", ctypes.c_int64, [ctypes.c_void_p, ctypes.POINTER(f32p), i64p,
                                                      ctypes.POINTER(ctypes.c_int)]),
            ("rgref_program_op_macs", ctypes.c_int64, [ctypes.c_void_p, ctypes.c_int64]),
            ("rgref_program_total_macs", ctypes.c_int64, [ctypes.c_void_p]),
            ("rgref_last_error", ctypes.c_char_p, []),
            ("rgref_set_threads", None, [ctypes.c_int]),
            ("rgref_get_threads", ctypes.c_int, []),
        ]
        for name, res, args in sig:
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    return a.ctypes.data_as(f32p)


# ---- primitives ------------------------------------------------------------
def manual_seed(seed: int) -> None:
    lib().rgref_manual_seed(seed & 0xFFFFFFFFFFFFFFFF)


def fill(kind: str, shape, lo: float = 0.0, hi: float = 1.0) -> np.ndarray:
    a = np.empty(shape, np.float32)
    if kind == "uniform":
        lib().rgref_fill_uniform(_fp(a), a.size)
    elif kind == "range":
        lib().rgref_fill_uniform_range(_fp(a), a.size, lo, hi)
    else:
        lib().rgref_fill_normal(_fp(a), a.size)
    return a


def quantize(v: np.ndarray):
    v = np.ascontiguousarray(v, np.float32).reshape(-1)
    q = np.empty(v.size, np.int8)
    s = lib().rgref_quantize(_fp(v), v.size, q.ctypes.data_as(i8p))
    return q, np.float32(s)


def act_apply(code: int, param: float, x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32).reshape(-1)
    y = np.empty_like(x)
    lib().rgref_act_apply_array(code, param, _fp(x), _fp(y), x.size)
    return y


def gemm_fused(a_q, a_scale, b_q, b_scale, m, k, n, bias, act=0, param=0.0, parallel=False):
    a_q = np.ascontiguousarray(a_q, np.int8)
    b_q = np.ascontiguousarray(b_q, np.int8)
    bias = np.ascontiguousarray(bias, np.float32)
    out = np.empty(m * n, np.float32)
    acc = np.empty(m * n, np.int32)
    lib().rgref_int8_gemm_fused(a_q.ctypes.data_as(i8p), a_scale, b_q.ctypes.data_as(i8p), b_scale, m, k, n,
                                _fp(bias), act, param, _fp(out), acc.ctypes.data_as(i32p), 1 if parallel else 0)
    return out.reshape(m, n), acc.reshape(m, n)


def im2col(x, c, h, w, k, stride, pad):
    oh = lib().rgref_out_size(h, k, stride, pad)
    ow = lib().rgref_out_size(w, k, stride, pad)
    x = np.ascontiguousarray(x, np.float32)
    cols = np.empty(c * k * k * oh * ow, np.float32)
    lib().rgref_im2col(_fp(x), c, h, w, k, stride, pad, oh, ow, _fp(cols))
    return cols.reshape(c * k * k, oh * ow)


def max_pool2d(x, n, c, h, w, k, stride):
    oh = lib().rgref_out_size(h, k, stride, 0)
    ow = lib().rgref_out_size(w, k, stride, 0)
    x = np.ascontiguousarray(x, np.float32)
    out = np.empty(n * c * oh * ow, np.float32)
    lib().rgref_max_pool2d(_fp(x), n, c, h, w, k, stride, _fp(out), 0)
    return out.reshape(n, c, oh, ow)


def softmax_rows(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, np.float32)
    y = np.empty_like(x)
    last = x.shape[-1]
    lib().rgref_softmax_rows(_fp(x), x.size // last, last, _fp(y))
    return y


# ---- programs ----------------------------------------------------------------
def to_ref_layers(layers: Sequence) -> tuple:
    """LayerSpec objects (rustgears_amd.inference.LayerSpec) -> rgref_layer[]."""
    arr = (RefLayer * max(1, len(layers)))()
    keep: List[np.ndarray] = []
    for i, l in enumerate(layers):
        c = arr[i]
        name = type(l).__name__
        if name == "Linear":
            c.kind = 1
            c.in_features, c.out_features = l.in_features, l.out_features
            w, b = np.ascontiguousarray(l.weight, np.float32), np.ascontiguousarray(l.bias, np.float32)
            c.weight, c.weight_len, c.bias, c.bias_len = _fp(w), w.size, _fp(b), b.size
            keep += [w, b]
        elif name == "Conv2d":
            c.kind = 2
            c.in_channels, c.out_channels, c.kernel = l.in_channels, l.out_channels, l.kernel
            c.stride, c.padding = l.stride, l.padding
            w, b = np.ascontiguousarray(l.weight, np.float32), np.ascontiguousarray(l.bias, np.float32)
            c.weight, c.weight_len, c.bias, c.bias_len = _fp(w), w.size, _fp(b), b.size
            keep += [w, b]
        elif name == "ChannelAffine":
            c.kind = 3
            s, t = np.ascontiguousarray(l.scale, np.float32), np.ascontiguousarray(l.shift, np.float32)
            # fold_batch_norm and the lone affine index shift[c] for every
            # c < scale.len() (mod.rs:236-237, 246; npu.rs:254-268): a shorter
            # shift is an index panic there, a longer one is read no further
            if t.size < s.size:
                raise ValueError("ChannelAffine: shift shorter than scale (the reference panics)")
            c.scale, c.shift, c.affine_len = _fp(s), _fp(t), s.size
            keep += [s, t]
        elif name == "MaxPool2d":
            c.kind = 4
            c.pool_kernel, c.pool_stride = l.kernel, l.stride
        elif name == "Flatten":
            c.kind = 5
        elif name == "Activation":
            c.kind = 6
            c.act, c.act_param = l.act.code, l.act.param
        elif name == "Softmax":
            c.kind = 7
        else:
            raise TypeError(name)
    return arr, keep


INT8, FP16, FP32 = 0, 1, 2  # NpuPrecision (npu.rs:25-30); FP32 = the standard path (run_standard, mod.rs:260-331)


def round_fp16(x) -> np.ndarray:
    """round_fp16 (quantize.rs:50-64), elementwise."""
    a = np.ascontiguousarray(np.asarray(x, np.float32))
    y = np.empty_like(a)
    lib().rgref_round_fp16_array(_fp(a), _fp(y), a.size)
    return y


def fp16_gemm_fused(a, b_t, bias, act: int = 0, param: float = 0.0) -> np.ndarray:
    """fp16_gemm_fused (npu.rs:425-445): a [m,k] f32, b_t [n,k] f32 (already
    fp16-rounded), bias [n]."""
    a = np.ascontiguousarray(a, np.float32)
    b_t = np.ascontiguousarray(b_t, np.float32)
    bias = np.ascontiguousarray(bias, np.float32)
    m, k = a.shape
    n = b_t.shape[0]
    out = np.empty((m, n), np.float32)
    lib().rgref_fp16_gemm_fused(_fp(a), _fp(b_t), m, k, n, _fp(bias), act, param, _fp(out), 0)
    return out


class RefProgram:
    """npu::compile + NpuProgram::execute restated on the CPU, for
    NpuPrecision::Int8 (precision=INT8) or ::Fp16 (precision=FP16)."""

    def __init__(self, layers: Sequence, precision: int = INT8):
        arr, keep = to_ref_layers(layers)
        self._p = lib().rgref_compile_precision(arr, len(layers), precision)
        self.precision = precision
        del keep

    def __del__(self):
        if getattr(self, "_p", None):
            lib().rgref_program_free(self._p)
            self._p = None

    @property
    def num_ops(self) -> int:
        return lib().rgref_program_num_ops(self._p)

    @property
    def fp32_bytes(self) -> int:
        return lib().rgref_program_fp32_bytes(self._p)

    @property
    def npu_bytes(self) -> int:
        return lib().rgref_program_npu_bytes(self._p)

    @property
    def original_layers(self) -> int:
        return lib().rgref_program_original_layers(self._p)

    def labels(self) -> List[str]:
        out = []
        for i in range(self.num_ops):
            buf = ctypes.create_string_buffer(256)
            lib().rgref_program_op_label(self._p, i, buf, 256)
            out.append(buf.value.decode())
        return out

    def op_weight(self, i: int):
        w = i8p()
        s = ctypes.c_float()
        b = f32p()
        n = lib().rgref_program_op_weight(self._p, i, ctypes.byref(w), ctypes.byref(s), ctypes.byref(b))
        if n <= 0 or not w:
            return np.zeros(0, np.int8), np.float32(s.value)
        return np.ctypeslib.as_array(w, shape=(n,)).copy(), np.float32(s.value)

    def op_weight_fp16(self, i: int) -> np.ndarray:
        """FP16 program: op i's round_fp16 weights as [out, K] f32."""
        w = f32p()
        rows = ctypes.c_int64()
        n = lib().rgref_program_op_weight_fp16(self._p, i, ctypes.byref(w), ctypes.byref(rows))
        if n <= 0 or not w:
            return np.zeros((0, 0), np.float32)
        return np.ctypeslib.as_array(w, shape=(n,)).copy().reshape(rows.value, n // rows.value)

    def set_capture(self, on: bool) -> None:
        lib().rgref_program_set_capture(self._p, 1 if on else 0)

    def capture(self, op: int, what: int) -> np.ndarray:
        p = ctypes.c_void_p()
        n = lib().rgref_program_capture(self._p, op, what, ctypes.byref(p))
        dt = {CAP_QACT: np.int8, CAP_SCALE: np.float32, CAP_ACC: np.int32, CAP_OUT: np.float32}[what]
        if n <= 0 or not p.value:
            return np.zeros(0, dt)
        buf = (ctypes.c_char * (n * np.dtype(dt).itemsize)).from_address(p.value)
        return np.frombuffer(bytes(buf), dtype=dt).copy()

    def run(self, x: np.ndarray, parallel: bool = False) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        sh = (ctypes.c_int64 * max(1, x.ndim))(*x.shape)
        st = lib().rgref_execute(self._p, _fp(x), sh, x.ndim, 1 if parallel else 0)
        if st != 0:
            raise ValueError(lib().rgref_last_error().decode())
        y = f32p()
        shape = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int()
        n = lib().rgref_program_output(self._p, ctypes.byref(y), shape, ctypes.byref(nd))
        out = np.ctypeslib.as_array(y, shape=(n,)).copy() if n > 0 else np.zeros(0, np.float32)
        return out.reshape(tuple(shape[i] for i in range(nd.value)))

    def op_macs(self, i: int) -> int:
        return lib().rgref_program_op_macs(self._p, i)

    @property
    def total_macs(self) -> int:
        return lib().rgref_program_total_macs(self._p)


def set_threads(n: int) -> None:
    lib().rgref_set_threads(int(n))


def get_threads() -> int:
    return lib().rgref_get_threads()
