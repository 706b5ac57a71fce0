"""Seeded synthetic data with the reference's generator (src/rng.rs:10-98).

The generator lives in librgnpu (rng.cpp).  Arrays come back as float32 in
the reference's draw order: Tensor::rand -> uniform, Tensor::uniform(lo, hi)
-> lo + (hi-lo)*u, Tensor::randn -> Box-Muller (src/tensor/mod.rs:116-131).
"""
from __future__ import annotations

import numpy as np

from . import _native as N


def manual_seed(seed: int) -> None:
    """rng.rs:71-73."""
    N.lib().rgnpu_manual_seed(int(seed) & 0xFFFFFFFFFFFFFFFF)


def _alloc(shape) -> np.ndarray:
    return np.empty(tuple(int(s) for s in shape), dtype=np.float32)


def rand(shape) -> np.ndarray:
    """Tensor::rand (tensor/mod.rs:122-125): U[0, 1)."""
    a = _alloc(shape)
    N.lib().rgnpu_fill_uniform(a.ctypes.data_as(N.f32p), a.size)
    return a


def uniform(shape, lo: float, hi: float) -> np.ndarray:
    """Tensor::uniform (tensor/mod.rs:128-131): U[lo, hi)."""
    a = _alloc(shape)
    N.lib().rgnpu_fill_uniform_range(a.ctypes.data_as(N.f32p), a.size, float(np.float32(lo)), float(np.float32(hi)))
    return a


def randn(shape) -> np.ndarray:
    """Tensor::randn (tensor/mod.rs:116-119): Box-Muller N(0, 1)."""
    a = _alloc(shape)
    N.lib().rgnpu_fill_normal(a.ctypes.data_as(N.f32p), a.size)
    return a
