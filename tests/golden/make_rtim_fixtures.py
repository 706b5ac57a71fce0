"""Writes the RTIM byte fixtures (tests/golden/rtim_*.rtim) and their expected
decodings (tests/golden/rtim_cases.json).

Each file is assembled field by field from literal little-endian hex, read off
the reference's writer and reader (src/save.rs:172-224 save_layers,
src/save.rs:227-279 load_inference_layers, src/save.rs:35-75 for the u32 /
f32 / length-prefixed f32-vector encodings).  Nothing here calls the product
or the oracle, so the fixtures pin both:
  * the product's rgnpu_rtim_save must write exactly the canonical files;
  * rgnpu_rtim_load (and the oracle's restatement) must decode every file to
    the layers listed in rtim_cases.json, or fail with the listed error kind
    (InvalidData = RGNPU_ERR_FORMAT, UnexpectedEof = RGNPU_ERR_IO).

Run:  python tests/golden/make_rtim_fixtures.py
"""
import json
import os

HERE = os.path.dirname(os.path.abspath(__file__))

# Field encodings used below, written out once:
#   u32 1 = 01000000, u32 2 = 02000000, ... (save.rs:35-37, to_le_bytes)
#   f32 values by their IEEE-754 bits, little-endian (save.rs:47-49):
#     0.5 = 0x3f000000 -> 0000003f     -1.5 = 0xbfc00000 -> 0000c0bf
#     2.0 = 0x40000000 -> 00000040      0.25 = 0x3e800000 -> 0000803e
#     -0.0 = 0x80000000 -> 00000080     1.0 = 0x3f800000 -> 0000803f
#     0.125 = 0x3e000000 -> 0000003e    3.0 = 0x40400000 -> 00004040
#     7.0 = 0x40e00000 -> 0000e040      -2.0 = 0xc0000000 -> 000000c0
#   f32 vector = u32 length, then the values (save.rs:59-65)

MAGIC = "5254494d"  # b"RTIM" (save.rs:17)


def hexbytes(parts):
    return bytes.fromhex("".join(h for h, _ in parts))


CASES = {}

# --- every tag (1..7) and every activation code (0..5) ----------------------
all_tags = [
    (MAGIC, "magic RTIM"),
    ("0c000000", "count = 12 layers"),
    # Linear { in 2, out 3, weight [6], bias [3] }  (save.rs:178-184)
    ("01000000", "tag 1 Linear"), ("02000000", "in_features 2"), ("03000000", "out_features 3"),
    ("06000000", "weight len 6"),
    ("0000003f", "0.5"), ("0000c0bf", "-1.5"), ("00000040", "2.0"),
    ("0000803e", "0.25"), ("00000080", "-0.0"), ("0000803f", "1.0"),
    ("03000000", "bias len 3"), ("0000003e", "0.125"), ("00004040", "3.0"), ("000000c0", "-2.0"),
    # Conv2d { in 1, out 2, k 1, s 2, p 1, weight [2], bias [2] }  (save.rs:185-194)
    ("02000000", "tag 2 Conv2d"), ("01000000", "in_channels 1"), ("02000000", "out_channels 2"),
    ("01000000", "kernel 1"), ("02000000", "stride 2"), ("01000000", "padding 1"),
    ("02000000", "weight len 2"), ("0000803f", "1.0"), ("000000c0", "-2.0"),
    ("02000000", "bias len 2"), ("0000003f", "0.5"), ("00000080", "-0.0"),
    # ChannelAffine { scale [2], shift [2] }  (save.rs:195-199)
    ("03000000", "tag 3 ChannelAffine"),
    ("02000000", "scale len 2"), ("00000040", "2.0"), ("0000803e", "0.25"),
    ("02000000", "shift len 2"), ("0000c0bf", "-1.5"), ("0000003e", "0.125"),
    # MaxPool2d { kernel 3, stride 2 }  (save.rs:200-204)
    ("04000000", "tag 4 MaxPool2d"), ("03000000", "kernel 3"), ("02000000", "stride 2"),
    # Flatten  (save.rs:205)
    ("05000000", "tag 5 Flatten"),
    # Activation codes 0..5, param 0.0 except LeakyReLU's slope (save.rs:206-218)
    ("06000000", "tag 6"), ("00000000", "code 0 None"), ("00000000", "param 0.0"),
    ("06000000", "tag 6"), ("01000000", "code 1 ReLU"), ("00000000", "param 0.0"),
    ("06000000", "tag 6"), ("02000000", "code 2 Sigmoid"), ("00000000", "param 0.0"),
    ("06000000", "tag 6"), ("03000000", "code 3 Tanh"), ("00000000", "param 0.0"),
    ("06000000", "tag 6"), ("04000000", "code 4 GELU"), ("00000000", "param 0.0"),
    ("06000000", "tag 6"), ("05000000", "code 5 LeakyReLU"), ("0000003e", "param 0.125"),
    # Softmax  (save.rs:219)
    ("07000000", "tag 7 Softmax"),
]
CASES["rtim_all_tags"] = dict(parts=all_tags, canonical=True, layers=[
    {"kind": "Linear", "in_features": 2, "out_features": 3,
     "weight": ["3f000000", "bfc00000", "40000000", "3e800000", "80000000", "3f800000"],
     "bias": ["3e000000", "40400000", "c0000000"]},
    {"kind": "Conv2d", "in_channels": 1, "out_channels": 2, "kernel": 1, "stride": 2, "padding": 1,
     "weight": ["3f800000", "c0000000"], "bias": ["3f000000", "80000000"]},
    {"kind": "ChannelAffine", "scale": ["40000000", "3e800000"], "shift": ["bfc00000", "3e000000"]},
    {"kind": "MaxPool2d", "kernel": 3, "stride": 2},
    {"kind": "Flatten"},
    {"kind": "Activation", "code": 0, "param": "00000000"},
    {"kind": "Activation", "code": 1, "param": "00000000"},
    {"kind": "Activation", "code": 2, "param": "00000000"},
    {"kind": "Activation", "code": 3, "param": "00000000"},
    {"kind": "Activation", "code": 4, "param": "00000000"},
    {"kind": "Activation", "code": 5, "param": "3e000000"},
    {"kind": "Softmax"},
])

# --- empty model ------------------------------------------------------------
CASES["rtim_empty"] = dict(parts=[(MAGIC, "magic"), ("00000000", "count 0")], canonical=True, layers=[])

# --- ChannelAffine whose shift is longer than its scale: loaded as is -------
# (save.rs:254 reads two independent vectors and compares nothing)
CASES["rtim_affine_lengths_differ"] = dict(parts=[
    (MAGIC, "magic"), ("01000000", "count 1"),
    ("03000000", "tag 3"), ("02000000", "scale len 2"), ("0000803f", "1.0"), ("00000040", "2.0"),
    ("03000000", "shift len 3"), ("0000003f", "0.5"), ("0000c0bf", "-1.5"), ("0000e040", "7.0"),
], canonical=True, layers=[
    {"kind": "ChannelAffine", "scale": ["3f800000", "40000000"], "shift": ["3f000000", "bfc00000", "40e00000"]},
])

# --- u32 fields above 2^31 read back unchanged (usize in the reference) ------
CASES["rtim_u32_fields"] = dict(parts=[
    (MAGIC, "magic"), ("02000000", "count 2"),
    ("01000000", "tag 1"), ("01000080", "in 0x80000001"), ("ffffffff", "out 0xffffffff"),
    ("00000000", "weight len 0"), ("00000000", "bias len 0"),
    ("04000000", "tag 4"), ("feffffff", "kernel 0xfffffffe"), ("00000080", "stride 0x80000000"),
], canonical=True, layers=[
    {"kind": "Linear", "in_features": 0x80000001, "out_features": 0xFFFFFFFF, "weight": [], "bias": []},
    {"kind": "MaxPool2d", "kernel": 0xFFFFFFFE, "stride": 0x80000000},
])

# --- a non-LeakyReLU code with a nonzero param: the param is dropped ---------
# (save.rs:259-266 uses p only for code 5); saving writes 0.0, so the file is
# not canonical
CASES["rtim_param_ignored"] = dict(parts=[
    (MAGIC, "magic"), ("01000000", "count 1"),
    ("06000000", "tag 6"), ("01000000", "code 1 ReLU"), ("0000e040", "param 7.0"),
], canonical=False, layers=[{"kind": "Activation", "code": 1, "param": "00000000"}])

# --- errors -----------------------------------------------------------------
CASES["rtim_bad_magic"] = dict(parts=[("5254494e", "RTIN"), ("00000000", "count 0")], canonical=False,
                               error="InvalidData", message="invalid RTIM model header")
CASES["rtim_unknown_tag"] = dict(parts=[(MAGIC, "magic"), ("01000000", "count 1"), ("08000000", "tag 8")],
                                 canonical=False, error="InvalidData", message="unknown layer tag 8")
CASES["rtim_unknown_activation"] = dict(parts=[
    (MAGIC, "magic"), ("01000000", "count 1"), ("06000000", "tag 6"), ("06000000", "code 6"),
    ("00000000", "param")], canonical=False, error="InvalidData", message="unknown activation tag 6")
CASES["rtim_truncated_vector"] = dict(parts=[
    (MAGIC, "magic"), ("01000000", "count 1"), ("03000000", "tag 3"), ("03000000", "scale len 3"),
    ("0000803f", "1.0"), ("00000040", "2.0")], canonical=False, error="UnexpectedEof")
CASES["rtim_count_too_large"] = dict(parts=[
    (MAGIC, "magic"), ("02000000", "count 2"), ("05000000", "tag 5 Flatten")],
    canonical=False, error="UnexpectedEof")
CASES["rtim_short_header"] = dict(parts=[("525449", "RTI")], canonical=False, error="UnexpectedEof")


def main():
    assert len(CASES["rtim_all_tags"]["layers"]) == int.from_bytes(bytes.fromhex(all_tags[1][0]), "little")
    index = {}
    for name, c in CASES.items():
        data = hexbytes(c["parts"])
        with open(os.path.join(HERE, name + ".rtim"), "wb") as f:
            f.write(data)
        entry = {"canonical": c["canonical"], "bytes": len(data)}
        if "layers" in c:
            entry["layers"] = c["layers"]
        else:
            entry["error"] = c["error"]
            if "message" in c:
                entry["message"] = c["message"]
        index[name] = entry
    with open(os.path.join(HERE, "rtim_cases.json"), "w") as f:
        json.dump(index, f, indent=1, sort_keys=True)
        f.write("\n")


if __name__ == "__main__":
    main()
