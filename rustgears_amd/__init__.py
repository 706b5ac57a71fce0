"""rustgears_amd — MI355X-native INT8 execution provider for RustGears'
InferenceSession (elandice/RustGears), with the reference's Python-side API
mirror: LayerSpec IR, InferenceSession, NpuProfile, RTIM and seeded data.
The compute path is librgnpu.so (HIP, gfx950); see include/rgnpu.h.
"""
from ._native import RgnpuError, device_count, lib
from .inference import (Activation, DeviceBuffer, ExecutionProvider, InferenceSession, LayerSpec, NpuPrecision,
                        NpuProfile, OpRecord)
from .rng import manual_seed, rand, randn, uniform
from .save import load_inference_layers, save_inference_model, save_layers

__all__ = [
    "Activation", "DeviceBuffer", "ExecutionProvider", "InferenceSession", "LayerSpec", "NpuPrecision", "NpuProfile",
    "OpRecord", "RgnpuError", "device_count", "lib", "load_inference_layers", "manual_seed", "rand", "randn",
    "save_inference_model", "save_layers", "uniform",
]
