import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through librgnpu on the GPU)")


@pytest.fixture(scope="session")
def ref():
    import oracle
    oracle.lib()
    return oracle


@pytest.fixture(scope="session")
def rg():
    import rustgears_amd
    rustgears_amd.lib()
    return rustgears_amd


def f32_bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bitexact_f32(a, b, what=""):
    a = np.ascontiguousarray(a, np.float32).reshape(-1)
    b = np.ascontiguousarray(b, np.float32).reshape(-1)
    assert a.shape == b.shape, f"{what}: shape {a.shape} vs {b.shape}"
    same = (a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))
    if not same.all():
        idx = np.flatnonzero(~same)[:5]
        raise AssertionError(f"{what}: {np.count_nonzero(~same)} of {a.size} f32 differ, e.g. "
                             f"{[(int(i), float(a[i]), float(b[i])) for i in idx]}")


def round_half_away(x):
    """f32::round on float32 arrays, exact: trunc, then away from zero when
    the dropped fraction is >= 0.5 (the subtraction x - trunc(x) is exact)."""
    x = np.asarray(x, np.float32)
    t = np.trunc(x)
    frac = np.abs(x - t)
    return (t + np.where(frac >= np.float32(0.5), np.sign(x), np.float32(0))).astype(np.float32)


def quantize_np(v):
    """QuantTensor::from_f32 (quantize.rs:18-24) in numpy, used to check
    captured activations at sizes where the C oracle is too slow."""
    v = np.asarray(v, np.float32).reshape(-1)
    a = np.abs(v)
    a = a[~np.isnan(a)]
    max_abs = np.float32(a.max()) if a.size else np.float32(0)
    scale = np.float32(1.0) if max_abs < np.float32(1e-12) else np.float32(max_abs / np.float32(127.0))
    inv = np.float32(np.float32(1.0) / scale)
    with np.errstate(invalid="ignore"):
        r = round_half_away((v * inv).astype(np.float32))
        r = np.clip(r, -127, 127)
        r = np.where(np.isnan(r), 0, r)
    return r.astype(np.int8), scale
