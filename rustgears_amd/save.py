"""RTIM portable inference graph (src/save.rs:165-279) through librgnpu."""
from __future__ import annotations

import ctypes
import os
from typing import List, Sequence

from . import _native as N
from .inference import AnyLayer, from_c_layers, to_c_layers


def save_layers(layers: Sequence[AnyLayer], path) -> None:
    """save_layers (save.rs:172-224), atomic replace."""
    arr, keep = to_c_layers(layers)
    N.check(N.lib().rgnpu_rtim_save(os.fsencode(path), arr, len(layers)))
    del keep


def save_inference_model(module, path) -> None:
    """save_inference_model (save.rs:165-169)."""
    module.eval()
    save_layers(module.export(), path)


def load_inference_layers(path) -> List[AnyLayer]:
    """load_inference_layers (save.rs:227-279).  Raises RgnpuError with code
    ERR_FORMAT for InvalidData and ERR_IO for I/O failures."""
    h = ctypes.c_void_p()
    ptr = ctypes.POINTER(N.CLayer)()
    n = ctypes.c_int64()
    N.check(N.lib().rgnpu_rtim_load(os.fsencode(path), ctypes.byref(h), ctypes.byref(ptr), ctypes.byref(n)))
    try:
        return from_c_layers(ptr, n.value)
    finally:
        N.lib().rgnpu_rtim_free(h)
