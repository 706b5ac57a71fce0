"""Modules whose constructors and export() produce the reference's LayerSpecs.

Mirrors the reference's seeded constructors and Module::export:
  init::{kaiming_uniform, xavier_uniform, normal, bias_uniform}  nn/init.rs:6-26
  Linear::new (W [in,out] then bias)                            nn/layers.rs:27-34, export 74-81
  Conv2d::new (W [out,in,k,k] then bias), stride/padding         nn/layers.rs:108-130, export 151-161
  MaxPool2d / Flatten / activations / Softmax exports           nn/layers.rs:263-376
  BatchNorm1d/2d defaults and export -> ChannelAffine           nn/norm.rs:53-66, 335-343
  Sequential::export                                             nn/mod.rs:204-210
Only inference export is provided (no forward/autograd).  Like the
reference, Silu has no export: Module.export raises ExportError.
"""
from __future__ import annotations

from typing import List

import numpy as np

from . import rng
from .inference import Activation, LayerSpec


class ExportError(RuntimeError):
    pass


f32 = np.float32


def kaiming_uniform(shape, fan_in: int) -> np.ndarray:
    bound = np.sqrt(f32(6.0) / f32(max(fan_in, 1)), dtype=f32)
    return rng.uniform(shape, -bound, bound)


def xavier_uniform(shape, fan_in: int, fan_out: int) -> np.ndarray:
    bound = np.sqrt(f32(6.0) / f32(max(fan_in + fan_out, 1)), dtype=f32)
    return rng.uniform(shape, -bound, bound)


def normal(shape, std: float) -> np.ndarray:
    return (rng.randn(shape) * f32(std)).astype(f32)


def bias_uniform(shape, fan_in: int) -> np.ndarray:
    bound = f32(1.0) / np.sqrt(f32(max(fan_in, 1)), dtype=f32)
    return rng.uniform(shape, -bound, bound)


class Module:
    def name(self) -> str:
        return "Module"

    def set_training(self, training: bool) -> None:
        pass

    def eval(self) -> None:
        self.set_training(False)

    def train(self) -> None:
        self.set_training(True)

    def export(self) -> List:
        raise ExportError(f"layer '{self.name()}' does not support export")


class Sequential(Module):
    def __init__(self):
        self.layers: List[Module] = []

    def add(self, layer: Module) -> "Sequential":
        self.layers.append(layer)
        return self

    def name(self) -> str:
        return f"Sequential[{len(self.layers)}]"

    def set_training(self, training: bool) -> None:
        for l in self.layers:
            l.set_training(training)

    def export(self) -> List:
        out = []
        for l in self.layers:
            out.extend(l.export())
        return out


class Linear(Module):
    def __init__(self, in_features: int, out_features: int, weight=None, bias=None):
        self.in_features, self.out_features = int(in_features), int(out_features)
        if weight is None:
            weight = kaiming_uniform([in_features, out_features], in_features)
            if bias is None:
                bias = bias_uniform([out_features], in_features)
        self.weight = np.asarray(weight, f32).reshape(in_features, out_features)
        self.bias = None if bias is None else np.asarray(bias, f32).reshape(out_features)

    @classmethod
    def xavier(cls, in_features: int, out_features: int) -> "Linear":
        """Build-defined init of the large configs: xavier W, then bias_uniform."""
        w = xavier_uniform([in_features, out_features], in_features, out_features)
        b = bias_uniform([out_features], in_features)
        return cls(in_features, out_features, w, b)

    def name(self) -> str:
        return f"Linear({self.in_features}, {self.out_features})"

    def export(self) -> List:
        bias = self.bias if self.bias is not None else np.zeros(self.out_features, f32)
        return [LayerSpec.Linear(self.in_features, self.out_features, self.weight.reshape(-1).copy(), bias.copy())]


class Conv2d(Module):
    def __init__(self, in_channels: int, out_channels: int, kernel_size: int, weight=None, bias=None):
        self.in_channels, self.out_channels, self.kernel_size = int(in_channels), int(out_channels), int(kernel_size)
        fan_in = in_channels * kernel_size * kernel_size
        if weight is None:
            weight = kaiming_uniform([out_channels, in_channels, kernel_size, kernel_size], fan_in)
            bias = bias_uniform([out_channels], fan_in)
        self.weight = np.asarray(weight, f32).reshape(out_channels, in_channels, kernel_size, kernel_size)
        self.bias = np.asarray(bias, f32).reshape(out_channels)
        self._stride, self._padding = 1, 0

    def stride(self, s: int) -> "Conv2d":
        self._stride = int(s)
        return self

    def padding(self, p: int) -> "Conv2d":
        self._padding = int(p)
        return self

    def name(self) -> str:
        return (f"Conv2d({self.in_channels}, {self.out_channels}, k={self.kernel_size}, "
                f"s={self._stride}, p={self._padding})")

    def export(self) -> List:
        return [LayerSpec.Conv2d(self.in_channels, self.out_channels, self.kernel_size, self._stride, self._padding,
                                 self.weight.reshape(-1).copy(), self.bias.copy())]


class BatchNorm(Module):
    def __init__(self, num_features: int, spatial: bool):
        if num_features <= 0:
            raise ValueError("BatchNorm feature count must be positive")
        self.num_features = int(num_features)
        self.gamma = np.ones(num_features, f32)
        self.beta = np.zeros(num_features, f32)
        self.running_mean = np.zeros(num_features, f32)
        self.running_var = np.ones(num_features, f32)
        self.eps = f32(1e-5)
        self.spatial = spatial
        self.training = True

    def set_training(self, training: bool) -> None:
        self.training = training

    def name(self) -> str:
        return f"BatchNorm{'2d' if self.spatial else '1d'}({self.num_features})"

    def export(self) -> List:
        # norm.rs:335-343: scale = g / sqrt(rv + eps) (division form), shift = b - rm*scale
        denom = np.sqrt((self.running_var + self.eps).astype(f32), dtype=f32)
        scale = (self.gamma / denom).astype(f32)
        shift = (self.beta - (self.running_mean * scale).astype(f32)).astype(f32)
        return [LayerSpec.ChannelAffine(scale, shift)]


class BatchNorm1d(BatchNorm):
    def __init__(self, num_features: int):
        super().__init__(num_features, False)


class BatchNorm2d(BatchNorm):
    def __init__(self, num_features: int):
        super().__init__(num_features, True)


class MaxPool2d(Module):
    def __init__(self, kernel: int, stride: int = None):
        self.kernel = int(kernel)
        self.stride = int(kernel if stride is None else stride)

    def name(self) -> str:
        return f"MaxPool2d(k={self.kernel}, s={self.stride})"

    def export(self) -> List:
        return [LayerSpec.MaxPool2d(self.kernel, self.stride)]


class Flatten(Module):
    def name(self) -> str:
        return "Flatten"

    def export(self) -> List:
        return [LayerSpec.Flatten()]


class _Act(Module):
    act = Activation.NONE
    label = "Act"

    def name(self) -> str:
        return self.label

    def export(self) -> List:
        return [LayerSpec.Activation(self.act)]


class Relu(_Act):
    act, label = Activation.RELU, "Relu"


class Sigmoid(_Act):
    act, label = Activation.SIGMOID, "Sigmoid"


class Tanh(_Act):
    act, label = Activation.TANH, "Tanh"


class Gelu(_Act):
    act, label = Activation.GELU, "Gelu"


class LeakyRelu(_Act):
    def __init__(self, slope: float):
        self.act = Activation.leaky_relu(slope)
        self.label = f"LeakyReLU({self.act.param})"


class Silu(Module):
    """nn::Silu has no export in the reference (layers.rs:338-347)."""

    def name(self) -> str:
        return "SiLU"


class Softmax(Module):
    def name(self) -> str:
        return "Softmax"

    def export(self) -> List:
        return [LayerSpec.Softmax()]
