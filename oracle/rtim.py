"""RTIM portable inference-model format, restated from the reference.

TEST INFRASTRUCTURE ONLY: imported by tests/, never by the product package.

Restates src/save.rs of elandice/RustGears:
  write_u32 / read_u32        save.rs:34-44   (little-endian u32)
  write_f32 / read_f32        save.rs:46-56   (little-endian IEEE-754 bits)
  write_f32_slice / read_f32_vec  save.rs:58-75 (u32 length, then the values)
  save_layers                 save.rs:172-224
  load_inference_layers       save.rs:227-279
Layers are dicts: {"kind": "Linear", "in_features", "out_features", "weight",
"bias"}, {"kind": "Conv2d", "in_channels", "out_channels", "kernel",
"stride", "padding", "weight", "bias"}, {"kind": "ChannelAffine", "scale",
"shift"}, {"kind": "MaxPool2d", "kernel", "stride"}, {"kind": "Flatten"},
{"kind": "Activation", "code", "param"}, {"kind": "Softmax"}; arrays are
float32 numpy vectors, sizes Python ints (the reference's usize).

Pinned by the hand-assembled byte fixtures of tests/golden/rtim_*.rtim
(tests/golden/make_rtim_fixtures.py), which spell every field out in hex.
"""
from __future__ import annotations

import struct
from typing import Dict, List

import numpy as np

MAGIC = b"RTIM"  # save.rs:17
TAGS = {"Linear": 1, "Conv2d": 2, "ChannelAffine": 3, "MaxPool2d": 4, "Flatten": 5, "Activation": 6,
        "Softmax": 7}  # save.rs:178-219


class RtimError(Exception):
    """io::Error of the reference: kind is "InvalidData" (bad magic, unknown
    tag or activation code) or "UnexpectedEof" (read_exact past the end)."""

    def __init__(self, kind: str, message: str = ""):
        super().__init__(f"{kind}: {message}")
        self.kind = kind
        self.message = message


def _u32(v: int) -> bytes:
    return struct.pack("<I", v & 0xFFFFFFFF)  # `as u32` truncates (save.rs:176, 180-181)


def _f32vec(a) -> bytes:
    a = np.ascontiguousarray(np.asarray(a, np.float32).reshape(-1))
    return _u32(a.size) + a.astype("<f4").tobytes()


def save_layers(layers: List[Dict]) -> bytes:
    """save_layers (save.rs:172-224) without the atomic file replace."""
    out = [MAGIC, _u32(len(layers))]
    for l in layers:
        k = l["kind"]
        out.append(_u32(TAGS[k]))
        if k == "Linear":
            out += [_u32(l["in_features"]), _u32(l["out_features"]), _f32vec(l["weight"]), _f32vec(l["bias"])]
        elif k == "Conv2d":
            out += [_u32(l[f]) for f in ("in_channels", "out_channels", "kernel", "stride", "padding")]
            out += [_f32vec(l["weight"]), _f32vec(l["bias"])]
        elif k == "ChannelAffine":
            out += [_f32vec(l["scale"]), _f32vec(l["shift"])]
        elif k == "MaxPool2d":
            out += [_u32(l["kernel"]), _u32(l["stride"])]
        elif k == "Activation":
            code = l["code"]
            if not 0 <= code <= 5:
                raise ValueError("Activation has no RTIM code (save.rs:207-214 covers codes 0..5)")
            param = np.float32(l["param"]) if code == 5 else np.float32(0.0)  # save.rs:208-213
            out += [_u32(code), struct.pack("<f", param)]
    return b"".join(out)


class _Reader:
    def __init__(self, data: bytes):
        self.data, self.pos = data, 0

    def take(self, n: int) -> bytes:
        if self.pos + n > len(self.data):
            raise RtimError("UnexpectedEof", "failed to fill whole buffer")
        b = self.data[self.pos:self.pos + n]
        self.pos += n
        return b

    def u32(self) -> int:
        return struct.unpack("<I", self.take(4))[0]

    def f32(self) -> np.float32:
        return np.frombuffer(self.take(4), "<f4")[0]

    def f32vec(self) -> np.ndarray:
        n = self.u32()  # read_f32_vec pushes one value at a time (save.rs:68-75)
        vals = [self.f32() for _ in range(n)]
        return np.array(vals, np.float32)


def load_layers(data: bytes) -> List[Dict]:
    """load_inference_layers (save.rs:227-279) on the file's bytes."""
    r = _Reader(data)
    if r.take(4) != MAGIC:
        raise RtimError("InvalidData", "invalid RTIM model header")
    count = r.u32()
    out: List[Dict] = []
    for _ in range(count):
        tag = r.u32()
        if tag == 1:
            l = {"kind": "Linear", "in_features": r.u32(), "out_features": r.u32()}
            l["weight"] = r.f32vec()
            l["bias"] = r.f32vec()
        elif tag == 2:
            l = {"kind": "Conv2d"}
            for f in ("in_channels", "out_channels", "kernel", "stride", "padding"):
                l[f] = r.u32()
            l["weight"] = r.f32vec()
            l["bias"] = r.f32vec()
        elif tag == 3:
            l = {"kind": "ChannelAffine", "scale": r.f32vec()}
            l["shift"] = r.f32vec()
        elif tag == 4:
            l = {"kind": "MaxPool2d", "kernel": r.u32()}
            l["stride"] = r.u32()
        elif tag == 5:
            l = {"kind": "Flatten"}
        elif tag == 6:
            code = r.u32()
            p = r.f32()
            if code > 5:
                raise RtimError("InvalidData", f"unknown activation tag {code}")
            l = {"kind": "Activation", "code": code, "param": p if code == 5 else np.float32(0.0)}
        elif tag == 7:
            l = {"kind": "Softmax"}
        else:
            raise RtimError("InvalidData", f"unknown layer tag {tag}")
        out.append(l)
    return out
