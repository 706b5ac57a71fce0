"""CPU-side checks of the product library and its host logic (no GPU calls).

* librgnpu.so loads and exports every function include/rgnpu.h declares.
* The product's seeded generator (rng.cpp) equals the oracle's, bit for bit.
* RTIM save/load (host-only code in librgnpu) round-trips and rejects what
  the reference rejects (save.rs:227-279, safetensors.rs:230-241).
* The device activation math (devmath.h) built for the host equals glibc on
  a strided sample of all f32 inputs.
* Without a GPU, program creation fails loudly instead of falling back.
"""
import ctypes
import os
import re
import struct
import subprocess

import numpy as np
import pytest

from conftest import ROOT, assert_bitexact_f32


def _declared_symbols():
    text = open(os.path.join(ROOT, "include", "rgnpu.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(rgnpu_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol(rg):
    lib = rg.lib()
    syms = _declared_symbols()
    assert len(syms) >= 25
    for s in syms:
        assert hasattr(lib, s), f"librgnpu.so does not export {s}"
    from rustgears_amd import _native
    assert sorted(n for n, _, _ in _native.SIGNATURES) == syms


def test_struct_layouts_match_header(rg, tmp_path):
    """ctypes mirrors of the ABI structs have the C compiler's sizes and
    field offsets."""
    from rustgears_amd import _native as N
    structs = {"rgnpu_layer": N.CLayer, "rgnpu_op_record": N.COpRecord, "rgnpu_profile": N.CProfile}
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "rgnpu.h"', "int main(void){"]
    for cname, py in structs.items():
        lines.append(f'printf("{cname} sizeof %zu\\n", sizeof({cname}));')
        for fname, _ in py._fields_:
            lines.append(f'printf("{cname} {fname} %zu\\n", offsetof({cname}, {fname}));')
    lines.append("return 0;}")
    src = tmp_path / "layout.c"
    src.write_text("\n".join(lines))
    exe = tmp_path / "layout"
    subprocess.run(["gcc", "-I", os.path.join(ROOT, "include"), "-o", str(exe), str(src)], check=True)
    for line in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.splitlines():
        cname, field, val = line.split()
        py = structs[cname]
        got = ctypes.sizeof(py) if field == "sizeof" else getattr(py, field).offset
        assert got == int(val), (cname, field, got, val)


@pytest.mark.parametrize("seed", [0, 42, 2026, 0xFFFFFFFFFFFFFFFF])
def test_product_rng_matches_oracle(ref, rg, seed):
    for kind in ("uniform", "range", "normal"):
        rg.manual_seed(seed)
        ref.manual_seed(seed)
        if kind == "uniform":
            a, b = rg.rand([3001]), ref.fill("uniform", [3001])
        elif kind == "range":
            a, b = rg.uniform([3001], -0.3, 0.7), ref.fill("range", [3001], -0.3, 0.7)
        else:
            a, b = rg.randn([3001]), ref.fill("normal", [3001])
        assert_bitexact_f32(a, b, f"{kind} seed {seed}")


def test_configs_draw_order_is_stable(rg):
    from rustgears_amd import configs
    m1, x1 = configs.quickstart()
    m2, x2 = configs.quickstart()
    assert np.array_equal(x1, x2)
    for a, b in zip(m1.export(), m2.export()):
        for f in ("weight", "bias", "scale", "shift"):
            if hasattr(a, f):
                assert np.array_equal(getattr(a, f), getattr(b, f))


def _layers_equal(a, b):
    assert len(a) == len(b)
    for x, y in zip(a, b):
        assert type(x) is type(y)
        for k, v in vars(x).items():
            w = getattr(y, k)
            if isinstance(v, np.ndarray):
                assert_bitexact_f32(v, w)
            else:
                assert v == w, (k, v, w)


def test_rtim_roundtrip(rg, tmp_path):
    from rustgears_amd import configs
    from rustgears_amd.inference import Activation, LayerSpec
    model, _ = configs.cnn(n=2, hw=8, c1=4, c2=8, fc=16)
    layers = model.export() + [LayerSpec.Activation(Activation.leaky_relu(0.25)), LayerSpec.Softmax(),
                               LayerSpec.Activation(Activation.GELU)]
    p = tmp_path / "m.rtim"
    rg.save_layers(layers, p)
    _layers_equal(layers, rg.load_inference_layers(p))
    # the byte stream follows save.rs:172-224: magic, count, tag of layer 0
    raw = p.read_bytes()
    assert raw[:4] == b"RTIM" and struct.unpack("<II", raw[4:12]) == (len(layers), 2)
    assert not [f for f in os.listdir(tmp_path) if f.startswith(".rtim-")]


def test_rtim_rejects_unknown_activation(rg, tmp_path):
    # safetensors.rs:230-241: tag 6 with activation code 99 -> InvalidData
    p = tmp_path / "bad.rtim"
    p.write_bytes(b"RTIM" + struct.pack("<III", 1, 6, 99) + struct.pack("<f", 0.0))
    with pytest.raises(rg.RgnpuError) as e:
        rg.load_inference_layers(p)
    assert e.value.code == 6 and "unknown activation tag 99" in str(e.value)


def test_rtim_silu_is_not_interchangeable(rg, tmp_path):
    # SiLU is this build's extension (layers.rs:341-343 has no export): the
    # reference reads activation codes 0..5 only (save.rs:259-267), so code 6
    # is InvalidData on load and a SiLU layer is refused on save.
    from rustgears_amd.inference import Activation, LayerSpec
    p = tmp_path / "silu.rtim"
    p.write_bytes(b"RTIM" + struct.pack("<III", 1, 6, 6) + struct.pack("<f", 0.0))
    with pytest.raises(rg.RgnpuError) as e:
        rg.load_inference_layers(p)
    assert e.value.code == 6 and "unknown activation tag 6" in str(e.value)
    q = tmp_path / "out.rtim"
    with pytest.raises(rg.RgnpuError) as e:
        rg.save_layers([LayerSpec.Activation(Activation.SILU)], q)
    assert e.value.code == 1 and "SiLU" in str(e.value)
    assert not q.exists() and not [f for f in os.listdir(tmp_path) if f.startswith(".rtim-")]


def test_rtim_rejects_bad_header_tag_and_truncation(rg, tmp_path):
    p = tmp_path / "x.rtim"
    p.write_bytes(b"RTIX" + struct.pack("<I", 0))
    with pytest.raises(rg.RgnpuError) as e:
        rg.load_inference_layers(p)
    assert e.value.code == 6
    p.write_bytes(b"RTIM" + struct.pack("<II", 1, 42))
    with pytest.raises(rg.RgnpuError) as e:
        rg.load_inference_layers(p)
    assert e.value.code == 6 and "unknown layer tag 42" in str(e.value)
    p.write_bytes(b"RTIM" + struct.pack("<III", 1, 1, 4))
    with pytest.raises(rg.RgnpuError) as e:
        rg.load_inference_layers(p)
    assert e.value.code == 5
    with pytest.raises(rg.RgnpuError):
        rg.load_inference_layers(tmp_path / "missing.rtim")


def test_silu_has_no_export_like_the_reference(rg):
    from rustgears_amd import nn
    with pytest.raises(nn.ExportError, match="layer 'SiLU' does not support export"):
        nn.Sequential().add(nn.Linear(2, 2)).add(nn.Silu()).export()


def test_batchnorm_export_division_form(rg):
    from rustgears_amd import nn
    bn = nn.BatchNorm1d(3)
    bn.gamma = np.array([1.0, 2.0, 0.5], np.float32)
    bn.beta = np.array([0.0, -1.0, 0.25], np.float32)
    bn.running_mean = np.array([0.1, 0.2, -0.3], np.float32)
    bn.running_var = np.array([1.0, 0.5, 2.0], np.float32)
    aff = bn.export()[0]
    for i in range(3):
        s = np.float32(bn.gamma[i] / np.float32(np.sqrt(np.float32(bn.running_var[i] + np.float32(1e-5)))))
        assert aff.scale[i] == s
        assert aff.shift[i] == np.float32(bn.beta[i] - np.float32(bn.running_mean[i] * s))


def test_devmath_matches_host_libm_sampled(tmp_path):
    """devmath.h (the GPU activation code) compiled for the host against
    glibc on every 61st f32 bit pattern (70M inputs, all binades).  The full
    2^32 sweep runs with RG_EXHAUSTIVE=1."""
    exe = tmp_path / "dmcheck"
    src = os.path.join(ROOT, "tests", "support", "devmath_host_check.cpp")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-o", str(exe), src, "-lm"],
                   check=True)
    stride = "1" if os.environ.get("RG_EXHAUSTIVE") == "1" else "61"
    out = subprocess.run([str(exe), stride, "0", str(min(8, os.cpu_count() or 1))], check=True, capture_output=True,
                         text=True).stdout
    rows = [l.split() for l in out.strip().splitlines()]
    assert [r[0] for r in rows] == ["tanhf", "expf", "sigmoid", "gelu", "silu", "tanhf_fast", "gelu_fast"]
    for name, checked, bad, first in rows:
        assert int(checked) > 60_000_000
        assert int(bad) == 0, f"{name}: {bad} mismatches vs libm, first input 0x{first}"


def test_fast_quantizer_matches_quantize_rule(tmp_path):
    """rgmath::quantize_rz, the fused requantization's quantizer (one add,
    a truncating saturating conversion and an integer clamp), against the rule
    of quantize.rs:22 (round half away from zero, clamp +-127, NaN -> 0) on
    every 13th f32 bit pattern; all 2^32 with RG_EXHAUSTIVE=1."""
    exe = tmp_path / "qcheck"
    src = os.path.join(ROOT, "tests", "support", "quant_host_check.cpp")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-o", str(exe), src], check=True)
    stride = "1" if os.environ.get("RG_EXHAUSTIVE") == "1" else "13"
    out = subprocess.run([str(exe), stride, "0", str(min(8, os.cpu_count() or 1))], check=True, capture_output=True,
                         text=True).stdout.split()
    assert int(out[0]) >= (1 << 32) // 13 and int(out[1]) == 0, f"first mismatch at 0x{out[2]}"
    # the clamp-free form: |v * inv| < 127.5 for every finite absmax (all of them)
    out = subprocess.run([str(exe), "1", "0", str(min(8, os.cpu_count() or 1)), "bound"], check=True,
                         capture_output=True, text=True).stdout.split()
    assert int(out[0]) == 0x7f800000 and int(out[1]) == 0, f"bound fails at absmax 0x{out[2]}"


def test_gelu_shape_for_certified_requantization(tmp_path):
    """The two properties of the exact f32 GELU (rgmath::gelu, equal to the
    reference's glibc form on every input) that let the INT8 GELU
    requantization take the tensor absmax from the largest pre-activation:
    it never decreases on [0, +inf], and |gelu(x)| <= kGeluNegAbsMax for every
    negative x, with equality at x = -0x1.8138e0p-1; and, for the certified
    FP16 hand-off, that fp16_bits(round_fp16(y)) is monotonic over the finite
    f32 values and never -0.  Every 16th block of 2^16 consecutive bit
    patterns (all of them with RG_EXHAUSTIVE=1)."""
    exe = tmp_path / "gshape"
    src = os.path.join(ROOT, "tests", "support", "gelu_shape_check.cpp")
    subprocess.run(["g++", "-O2", "-std=c++17", "-ffp-contract=off", "-pthread", "-o", str(exe), src, "-lm"],
                   check=True)
    stride = "1" if os.environ.get("RG_EXHAUSTIVE") == "1" else "16"
    out = subprocess.run([str(exe), str(min(8, os.cpu_count() or 1)), stride], check=True, capture_output=True,
                         text=True).stdout
    rows = {l.split()[0]: l.split()[1:] for l in out.strip().splitlines()}
    checked, bad, first = rows["monotone"]
    assert int(checked) >= 0x7f800000 // int(stride) - 65536 * 8
    assert int(bad) == 0, f"gelu decreases after input 0x{first}"
    checked, mx, arg, exceeds = rows["negmax"]
    assert int(exceeds) == 0, f"|gelu(0x{arg})| = 0x{mx} exceeds kGeluNegAbsMax"
    assert (mx, arg) == ("3e2e1f2c", "bf409c70")  # the bound is attained, at the argmax named in devmath.h
    checked, bad, first = rows["fp16mono"]
    assert int(checked) >= 0xff000000 // int(stride) - 65536 * 8
    assert int(bad) == 0, f"fp16_bits(round_fp16(y)) decreases (or gives -0) after input 0x{first}"


def test_program_create_fails_loudly_without_gpu(rg):
    if rg.device_count() > 0:
        pytest.skip("a GPU is present")
    from rustgears_amd import configs
    model, _ = configs.quickstart()
    with pytest.raises(rg.RgnpuError) as e:
        rg.InferenceSession.from_module(model, rg.ExecutionProvider.mi355x_int8())
    assert e.value.code == 3


def test_reference_providers_are_not_served_here(rg):
    from rustgears_amd import configs
    model, _ = configs.quickstart()
    with pytest.raises(NotImplementedError):
        rg.InferenceSession.from_module(model, rg.ExecutionProvider.npu_int8())
