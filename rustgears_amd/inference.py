"""InferenceSession API of RustGears, served by the MI355X INT8 provider.

Mirrors src/inference/mod.rs and src/inference/npu.rs of the reference:
  Activation            mod.rs:26-67
  LayerSpec             mod.rs:71-100
  ExecutionProvider     mod.rs:104-138 (+ the new Mi355x variant)
  NpuPrecision          npu.rs:25-39
  OpRecord/NpuProfile   npu.rs:109-176
  InferenceSession      mod.rs:146-222
Compilation and execution happen in librgnpu (C ABI, include/rgnpu.h); this
module converts arguments and results.  Tensors are numpy float32 arrays.
"""
from __future__ import annotations

import ctypes
import dataclasses
import enum
from typing import List, Optional, Sequence, Union

import numpy as np

from . import _native as N


# ---------------------------------------------------------------------------
# Activation (mod.rs:26-67)
# ---------------------------------------------------------------------------
def _rust_f32(v: float) -> str:
    """Rust's Display of an f32: shortest round-trip digits, positional."""
    f = np.float32(v)
    if np.isnan(f):
        return "NaN"
    if np.isinf(f):
        return "inf" if f > 0 else "-inf"
    s = np.format_float_positional(f, unique=True, trim="-")
    return s


@dataclasses.dataclass(frozen=True)
class Activation:
    code: int
    param: float = 0.0

    NONE: "Activation" = None  # type: ignore[assignment]
    RELU: "Activation" = None  # type: ignore[assignment]
    SIGMOID: "Activation" = None  # type: ignore[assignment]
    TANH: "Activation" = None  # type: ignore[assignment]
    GELU: "Activation" = None  # type: ignore[assignment]
    SILU: "Activation" = None  # type: ignore[assignment]

    @staticmethod
    def leaky_relu(slope: float) -> "Activation":
        return Activation(5, float(np.float32(slope)))

    def __str__(self) -> str:
        return {0: "none", 1: "ReLU", 2: "Sigmoid", 3: "Tanh", 4: "GELU", 6: "SiLU"}.get(
            self.code, f"LeakyReLU({_rust_f32(self.param)})" if self.code == 5 else "?")


Activation.NONE = Activation(0)
Activation.RELU = Activation(1)
Activation.SIGMOID = Activation(2)
Activation.TANH = Activation(3)
Activation.GELU = Activation(4)
Activation.SILU = Activation(6)  # extension: x * sigmoid(x) (nn/layers.rs:341-343)


# ---------------------------------------------------------------------------
# LayerSpec (mod.rs:71-100)
# ---------------------------------------------------------------------------
def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32).reshape(-1))


class LayerSpec:
    """Namespace of the LayerSpec variants."""

    @dataclasses.dataclass
    class Linear:
        in_features: int
        out_features: int
        weight: np.ndarray  # [in, out] row-major
        bias: np.ndarray

        def __post_init__(self):
            self.weight = _f32(self.weight)
            self.bias = _f32(self.bias)

    @dataclasses.dataclass
    class Conv2d:
        in_channels: int
        out_channels: int
        kernel: int
        stride: int
        padding: int
        weight: np.ndarray  # [out, in, k, k]
        bias: np.ndarray

        def __post_init__(self):
            self.weight = _f32(self.weight)
            self.bias = _f32(self.bias)

    @dataclasses.dataclass
    class ChannelAffine:
        scale: np.ndarray
        shift: np.ndarray

        def __post_init__(self):
            self.scale = _f32(self.scale)
            self.shift = _f32(self.shift)

    @dataclasses.dataclass
    class MaxPool2d:
        kernel: int
        stride: int

    @dataclasses.dataclass
    class Flatten:
        pass

    @dataclasses.dataclass
    class Activation:
        act: "Activation"

    @dataclasses.dataclass
    class Softmax:
        pass


AnyLayer = Union[LayerSpec.Linear, LayerSpec.Conv2d, LayerSpec.ChannelAffine, LayerSpec.MaxPool2d,
                 LayerSpec.Flatten, LayerSpec.Activation, LayerSpec.Softmax]


def _ptr(a: Optional[np.ndarray]):
    if a is None:
        return None
    return a.ctypes.data_as(N.f32p)


def to_c_layers(layers: Sequence[AnyLayer]):
    """Build an rgnpu_layer array; returns (array, keepalive list)."""
    arr = (N.CLayer * max(1, len(layers)))()
    keep = []
    for i, l in enumerate(layers):
        c = arr[i]
        if isinstance(l, LayerSpec.Linear):
            c.kind = N.LAYER_LINEAR
            c.in_features, c.out_features = int(l.in_features), int(l.out_features)
            c.weight, c.weight_len = _ptr(l.weight), l.weight.size
            c.bias, c.bias_len = _ptr(l.bias), l.bias.size
            keep += [l.weight, l.bias]
        elif isinstance(l, LayerSpec.Conv2d):
            c.kind = N.LAYER_CONV2D
            c.in_channels, c.out_channels = int(l.in_channels), int(l.out_channels)
            c.kernel, c.stride, c.padding = int(l.kernel), int(l.stride), int(l.padding)
            c.weight, c.weight_len = _ptr(l.weight), l.weight.size
            c.bias, c.bias_len = _ptr(l.bias), l.bias.size
            keep += [l.weight, l.bias]
        elif isinstance(l, LayerSpec.ChannelAffine):
            c.kind = N.LAYER_CHANNEL_AFFINE
            c.scale, c.scale_len = _ptr(l.scale), l.scale.size
            c.shift, c.shift_len = _ptr(l.shift), l.shift.size
            keep += [l.scale, l.shift]
        elif isinstance(l, LayerSpec.MaxPool2d):
            c.kind = N.LAYER_MAXPOOL2D
            c.pool_kernel, c.pool_stride = int(l.kernel), int(l.stride)
        elif isinstance(l, LayerSpec.Flatten):
            c.kind = N.LAYER_FLATTEN
        elif isinstance(l, LayerSpec.Activation):
            c.kind = N.LAYER_ACTIVATION
            c.act, c.act_param = int(l.act.code), float(l.act.param)
        elif isinstance(l, LayerSpec.Softmax):
            c.kind = N.LAYER_SOFTMAX
        else:
            raise TypeError(f"not a LayerSpec: {l!r}")
    return arr, keep


def from_c_layers(ptr, n: int) -> List[AnyLayer]:
    out: List[AnyLayer] = []
    for i in range(n):
        c = ptr[i]

        def vec(p, k):
            return np.ctypeslib.as_array(p, shape=(k,)).copy() if k else np.zeros(0, np.float32)

        if c.kind == N.LAYER_LINEAR:
            out.append(LayerSpec.Linear(c.in_features, c.out_features, vec(c.weight, c.weight_len),
                                        vec(c.bias, c.bias_len)))
        elif c.kind == N.LAYER_CONV2D:
            out.append(LayerSpec.Conv2d(c.in_channels, c.out_channels, c.kernel, c.stride, c.padding,
                                        vec(c.weight, c.weight_len), vec(c.bias, c.bias_len)))
        elif c.kind == N.LAYER_CHANNEL_AFFINE:
            out.append(LayerSpec.ChannelAffine(vec(c.scale, c.scale_len), vec(c.shift, c.shift_len)))
        elif c.kind == N.LAYER_MAXPOOL2D:
            out.append(LayerSpec.MaxPool2d(c.pool_kernel, c.pool_stride))
        elif c.kind == N.LAYER_FLATTEN:
            out.append(LayerSpec.Flatten())
        elif c.kind == N.LAYER_ACTIVATION:
            out.append(LayerSpec.Activation(Activation(int(c.act), float(c.act_param))))
        elif c.kind == N.LAYER_SOFTMAX:
            out.append(LayerSpec.Softmax())
    return out


# ---------------------------------------------------------------------------
# NpuPrecision / ExecutionProvider (npu.rs:25-39, mod.rs:104-138)
# ---------------------------------------------------------------------------
class NpuPrecision(enum.Enum):
    Int8 = 0
    Fp16 = 1

    def __str__(self) -> str:
        return "INT8" if self is NpuPrecision.Int8 else "FP16"


@dataclasses.dataclass(frozen=True)
class ExecutionProvider:
    """Provider selector.  `Mi355x(prec)` is the variant this package adds;
    the reference's own Cpu / Gpu(i) / Npu(prec) variants are listed so code
    can name them, but they run only in the reference."""

    kind: str
    precision: Optional[NpuPrecision] = None
    index: int = 0

    @staticmethod
    def Mi355x(precision: NpuPrecision = NpuPrecision.Int8, device: int = 0) -> "ExecutionProvider":
        return ExecutionProvider("mi355x", precision, device)

    @staticmethod
    def mi355x_int8(device: int = 0) -> "ExecutionProvider":
        return ExecutionProvider("mi355x", NpuPrecision.Int8, device)

    @staticmethod
    def mi355x_fp16(device: int = 0) -> "ExecutionProvider":
        return ExecutionProvider("mi355x", NpuPrecision.Fp16, device)

    @staticmethod
    def Gpu(index: int = 0) -> "ExecutionProvider":
        """ExecutionProvider::Gpu(i): the standard FP32 path (run_standard,
        mod.rs:260-331), executed on MI355X device `index`."""
        return ExecutionProvider("gpu", None, index)

    @staticmethod
    def Npu(precision: NpuPrecision) -> "ExecutionProvider":
        return ExecutionProvider("npu", precision)

    @staticmethod
    def npu_int8() -> "ExecutionProvider":
        return ExecutionProvider("npu", NpuPrecision.Int8)

    @staticmethod
    def npu_fp16() -> "ExecutionProvider":
        return ExecutionProvider("npu", NpuPrecision.Fp16)

    def __str__(self) -> str:
        if self.kind == "mi355x":
            return f"MI355X ({self.precision})"
        if self.kind == "npu":
            return f"NPU ({self.precision})"
        if self.kind == "gpu":
            return f"GPU:{self.index} (FP32)"
        return "CPU (FP32)"


# ---------------------------------------------------------------------------
# OpRecord / NpuProfile (npu.rs:109-176)
# ---------------------------------------------------------------------------
@dataclasses.dataclass
class OpRecord:
    op: str
    macs: int
    duration_ns: int
    kernel_ns: int


@dataclasses.dataclass
class NpuProfile:
    precision: NpuPrecision
    original_layers: int
    fused_ops: int
    fp32_weight_bytes: int
    npu_weight_bytes: int
    total_macs: int
    total_time_ns: int
    records: List[OpRecord]

    def compression_ratio(self) -> float:
        if self.npu_weight_bytes == 0:
            return 1.0
        return float(np.float32(self.fp32_weight_bytes) / np.float32(self.npu_weight_bytes))

    def gops(self) -> float:
        secs = max(self.total_time_ns / 1e9, 1e-9)
        return self.total_macs * 2.0 / secs / 1e9

    def __str__(self) -> str:
        head = (f"NPU Profile [{self.precision} | layers: {self.original_layers} -> {self.fused_ops} fused | "
                f"weights: {self.fp32_weight_bytes} B -> {self.npu_weight_bytes} B "
                f"({self.compression_ratio():.2f}x) | MACs: {self.total_macs} | "
                f"time: {self.total_time_ns / 1e3:.1f}µs ({self.gops():.2f} GOPS)]")
        lines = [head] + [f"  - {r.op:<42} {r.macs:>10} MACs   {r.duration_ns / 1e3:.1f}µs" for r in self.records]
        return "\n".join(lines) + "\n"


# ---------------------------------------------------------------------------
# device buffers (for device-resident runs)
# ---------------------------------------------------------------------------
class DeviceBuffer:
    """A hipMalloc'd buffer owned by Python (rgnpu_device_alloc)."""

    def __init__(self, nbytes: int, device: int = 0):
        p = ctypes.c_void_p()
        N.check(N.lib().rgnpu_device_alloc(device, int(nbytes), ctypes.byref(p)))
        self.ptr = p.value
        self.nbytes = int(nbytes)

    @classmethod
    def from_array(cls, a: np.ndarray, device: int = 0) -> "DeviceBuffer":
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes, device)
        b.upload(a)
        return b

    def upload(self, a: np.ndarray) -> None:
        a = np.ascontiguousarray(a)
        assert a.nbytes <= self.nbytes
        N.check(N.lib().rgnpu_memcpy_h2d(self.ptr, a.ctypes.data, a.nbytes))

    def download(self, shape, dtype=np.float32) -> np.ndarray:
        out = np.empty(shape, dtype=dtype)
        assert out.nbytes <= self.nbytes
        N.check(N.lib().rgnpu_memcpy_d2h(out.ctypes.data, self.ptr, out.nbytes))
        return out

    def free(self) -> None:
        if self.ptr:
            N.lib().rgnpu_device_free(self.ptr)
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


# ---------------------------------------------------------------------------
# InferenceSession (mod.rs:146-222)
# ---------------------------------------------------------------------------
class InferenceSession:
    def __init__(self, provider: ExecutionProvider, raw_layers: List[AnyLayer], handle: int):
        self._provider = provider
        self._raw_layers = raw_layers
        self._h = handle

    @classmethod
    def from_module(cls, model, provider: ExecutionProvider) -> "InferenceSession":
        """mod.rs:155-159: eval(), export(), then from_layers."""
        model.eval()
        layers = model.export()
        return cls.from_layers(layers, provider)

    @classmethod
    def from_layers(cls, raw_layers: Sequence[AnyLayer], provider: ExecutionProvider) -> "InferenceSession":
        """mod.rs:162-180 with the Mi355x variant -> rgnpu_program_create; the
        Gpu(i) variant builds the standard FP32 program on MI355X device i."""
        if provider.kind not in ("mi355x", "gpu"):
            raise NotImplementedError(
                f"provider {provider} runs in the reference; this package provides ExecutionProvider.Mi355x and Gpu")
        arr, keep = to_c_layers(raw_layers)
        h = ctypes.c_void_p()
        if provider.kind == "gpu":
            prec = N.PRECISION_FP32
        else:
            prec = N.PRECISION_INT8 if provider.precision is NpuPrecision.Int8 else N.PRECISION_FP16
        N.check(N.lib().rgnpu_program_create(arr, len(raw_layers), prec, provider.index, ctypes.byref(h)))
        del keep
        return cls(provider, list(raw_layers), h.value)

    def close(self) -> None:
        if self._h:
            N.lib().rgnpu_program_destroy(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def provider(self) -> ExecutionProvider:
        return self._provider

    def raw_layers(self) -> List[AnyLayer]:
        return self._raw_layers

    def compilation_report(self) -> str:
        n = N.lib().rgnpu_program_summary(self._h, None, 0)
        buf = ctypes.create_string_buffer(n + 1)
        N.lib().rgnpu_program_summary(self._h, buf, n + 1)
        return buf.value.decode()

    def op_labels(self) -> List[str]:
        labels = []
        for i in range(N.lib().rgnpu_program_num_ops(self._h)):
            buf = ctypes.create_string_buffer(128)
            N.lib().rgnpu_program_op_label(self._h, i, buf, 128)
            labels.append(buf.value.decode())
        return labels

    def op_weight(self, i: int):
        """(int8 weights [out,K] flat, scale) of op i as the reference holds them."""
        scale = ctypes.c_float()
        n = N.lib().rgnpu_program_op_weight(self._h, i, None, 0, ctypes.byref(scale))
        w = np.empty(max(n, 0), np.int8)
        N.lib().rgnpu_program_op_weight(self._h, i, w.ctypes.data, w.nbytes, ctypes.byref(scale))
        return w, np.float32(scale.value)

    def output_shape(self, shape) -> tuple:
        shp = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int32()
        sh = (ctypes.c_int64 * len(shape))(*shape)
        N.check(N.lib().rgnpu_program_run(self._h, None, sh, len(shape), None, 0, shp, ctypes.byref(nd)))
        return tuple(shp[i] for i in range(nd.value))

    def run(self, x: np.ndarray) -> np.ndarray:
        """mod.rs:212-221: host tensor in, host tensor out."""
        x = np.ascontiguousarray(x, dtype=np.float32)
        oshape = self.output_shape(x.shape)
        y = np.empty(oshape, np.float32)
        sh = (ctypes.c_int64 * max(1, x.ndim))(*x.shape)
        shp = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int32()
        N.check(N.lib().rgnpu_program_run(self._h, x.ctypes.data_as(N.f32p), sh, x.ndim,
                                          y.ctypes.data_as(N.f32p), y.size, shp, ctypes.byref(nd)))
        return y

    def run_device(self, d_x: DeviceBuffer, shape, d_y: DeviceBuffer) -> tuple:
        """Enqueue a device-resident run (asynchronous; see synchronize)."""
        sh = (ctypes.c_int64 * len(shape))(*shape)
        shp = (ctypes.c_int64 * 8)()
        nd = ctypes.c_int32()
        N.check(N.lib().rgnpu_program_run_device(self._h, d_x.ptr, sh, len(shape), d_y.ptr, d_y.nbytes // 4,
                                                 shp, ctypes.byref(nd)))
        return tuple(shp[i] for i in range(nd.value))

    def benchmark(self, d_x: DeviceBuffer, shape, d_y: DeviceBuffer, iters: int, per_kernel_events: bool = True,
                  evict_cache: bool = False):
        """rgnpu_program_benchmark: (total device ms, [OpRecord averages]).
        evict_cache: read 512 MiB of other data before each run, so that no run
        finds its weights in the 256 MB memory-side cache."""
        sh = (ctypes.c_int64 * len(shape))(*shape)
        ms = ctypes.c_double()
        recs = (N.COpRecord * 256)()
        flags = (1 if per_kernel_events else 0) | (2 if evict_cache else 0)
        N.check(N.lib().rgnpu_program_benchmark(self._h, d_x.ptr, sh, len(shape), d_y.ptr, d_y.nbytes // 4,
                                                int(iters), flags, ctypes.byref(ms),
                                                ctypes.cast(recs, ctypes.c_void_p), 256))
        n = N.lib().rgnpu_program_num_ops(self._h)
        return ms.value, [OpRecord(recs[i].op.decode(), int(recs[i].macs), int(recs[i].ns), int(recs[i].kernel_ns))
                          for i in range(n)]

    def synchronize(self) -> None:
        N.check(N.lib().rgnpu_program_synchronize(self._h))

    def set_profiling(self, level: int) -> None:
        N.check(N.lib().rgnpu_program_set_profiling(self._h, level))

    def barrier_stats(self) -> dict:
        """Cumulative barrier counters of the persistent grids over this
        session's contexts (rgnpu_program_barrier_stats): deferred and
        unsettled workgroups, finished barrier launches."""
        d, u, l = ctypes.c_uint64(), ctypes.c_uint64(), ctypes.c_uint64()
        N.check(N.lib().rgnpu_program_barrier_stats(self._h, ctypes.byref(d), ctypes.byref(u), ctypes.byref(l)))
        return {"deferred": d.value, "unsettled": u.value, "launches": l.value}

    def last_npu_profile(self) -> Optional[NpuProfile]:
        """mod.rs:193-195 (None for the standard FP32 path, which records no
        NPU profile)."""
        if self._provider.kind == "gpu":
            return None
        hdr = N.CProfile()
        recs = (N.COpRecord * 256)()
        st = N.lib().rgnpu_program_profile(self._h, ctypes.byref(hdr), recs, 256)
        if st != N.OK:
            return None
        records = [OpRecord(recs[i].op.decode(), int(recs[i].macs), int(recs[i].ns), int(recs[i].kernel_ns))
                   for i in range(hdr.n_records)]
        return NpuProfile(NpuPrecision(hdr.precision), hdr.original_layers, hdr.fused_ops, int(hdr.fp32_weight_bytes),
                          int(hdr.npu_weight_bytes), int(hdr.total_macs), int(hdr.total_ns), records)

    # ---- capture taps ------------------------------------------------------
    def set_capture(self, on) -> None:
        """True: capture taps (capture kernels: every op's i8 activations,
        scales, i32 sums and f32 output).  "production": production taps
        (the production kernels unchanged; what exists in memory between
        them is copied).  False: off."""
        mode = N.CAPTURE_PRODUCTION if on == "production" else (N.CAPTURE_FULL if on else N.CAPTURE_OFF)
        N.check(N.lib().rgnpu_program_set_capture(self._h, mode))

    def capture(self, op: int, what: int) -> np.ndarray:
        dtype = {N.CAP_QACT: np.int8, N.CAP_SCALE: np.float32, N.CAP_ACC: np.int32, N.CAP_OUT: np.float32}[what]
        n = N.lib().rgnpu_program_capture(self._h, op, what, None, 0)
        if n < 0:
            N.check(N.ERR_INVALID)
        out = np.empty(n, dtype)
        N.lib().rgnpu_program_capture(self._h, op, what, out.ctypes.data, out.nbytes)
        return out
