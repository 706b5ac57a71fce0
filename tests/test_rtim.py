"""RTIM portable inference model (src/save.rs:165-279).

CPU tests pin the byte format with the hand-assembled fixtures of
tests/golden/rtim_*.rtim (tests/golden/make_rtim_fixtures.py spells every
field out in hex from save.rs): the oracle's restatement (oracle/rtim.py) and
the product's reader/writer (librgnpu rgnpu_rtim_load / rgnpu_rtim_save) must
decode each file to the listed layers, or fail with the listed error, and
write the canonical files byte for byte.

The GPU test is the reference's own usage (examples/end_to_end.rs:103-112):
export a model, save it, load it back and run the loaded layers on the
MI355X INT8 provider; every op of the loaded model is compared bit for bit
with the oracle run on the original, never saved, layers.
"""
import json
import os

import numpy as np
import pytest

from conftest import assert_bitexact_f32

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
with open(os.path.join(GOLDEN, "rtim_cases.json")) as _f:
    CASES = json.load(_f)
ERR_IO, ERR_FORMAT, ERR_INVALID = 5, 6, 1
ERR_CODE = {"InvalidData": ERR_FORMAT, "UnexpectedEof": ERR_IO}


def _bits(hexes):
    return np.array([int(h, 16) for h in hexes], np.uint32).view(np.float32)


def _expected(case):
    """The fixture's layers as dicts with float32 arrays (oracle/rtim.py form)."""
    out = []
    for d in case["layers"]:
        d = dict(d)
        for k in ("weight", "bias", "scale", "shift"):
            if k in d:
                d[k] = _bits(d[k])
        if d["kind"] == "Activation":
            d["param"] = _bits([d["param"]])[0]
        out.append(d)
    return out


def _spec_from_dict(d):
    from rustgears_amd.inference import Activation, LayerSpec
    k = d["kind"]
    if k == "Linear":
        return LayerSpec.Linear(d["in_features"], d["out_features"], d["weight"], d["bias"])
    if k == "Conv2d":
        return LayerSpec.Conv2d(d["in_channels"], d["out_channels"], d["kernel"], d["stride"], d["padding"],
                                d["weight"], d["bias"])
    if k == "ChannelAffine":
        return LayerSpec.ChannelAffine(d["scale"], d["shift"])
    if k == "MaxPool2d":
        return LayerSpec.MaxPool2d(d["kernel"], d["stride"])
    if k == "Flatten":
        return LayerSpec.Flatten()
    if k == "Activation":
        return LayerSpec.Activation(Activation(int(d["code"]), float(d["param"])))
    return LayerSpec.Softmax()


def _dict_from_spec(l):
    k = type(l).__name__
    d = {"kind": k}
    if k == "Activation":
        d.update(code=l.act.code, param=np.float32(l.act.param))
    else:
        d.update({f: v for f, v in vars(l).items()})
    return d


def _same_layers(got, want, what):
    assert len(got) == len(want), what
    for i, (a, b) in enumerate(zip(got, want)):
        assert a.keys() == b.keys(), (what, i, a.keys(), b.keys())
        for f in a:
            if f in ("weight", "bias", "scale", "shift", "param"):
                x = np.atleast_1d(np.asarray(a[f], np.float32))
                y = np.atleast_1d(np.asarray(b[f], np.float32))
                assert x.view(np.uint32).tolist() == y.view(np.uint32).tolist(), (what, i, f)
            else:
                assert a[f] == b[f], (what, i, f, a[f], b[f])


def _fixture(name):
    with open(os.path.join(GOLDEN, name + ".rtim"), "rb") as f:
        return f.read()


@pytest.mark.parametrize("name", sorted(CASES))
def test_oracle_restatement_against_fixtures(name):
    from oracle import rtim
    case, data = CASES[name], _fixture(name)
    assert len(data) == case["bytes"]
    if "error" in case:
        with pytest.raises(rtim.RtimError) as e:
            rtim.load_layers(data)
        assert e.value.kind == case["error"]
        if "message" in case:
            assert e.value.message == case["message"]
        return
    want = _expected(case)
    _same_layers(rtim.load_layers(data), want, name)
    if case["canonical"]:
        assert rtim.save_layers(want) == data


@pytest.mark.parametrize("name", sorted(CASES))
def test_product_reader_against_fixtures(rg, name):
    case = CASES[name]
    path = os.path.join(GOLDEN, name + ".rtim")
    if "error" in case:
        with pytest.raises(rg.RgnpuError) as e:
            rg.load_inference_layers(path)
        assert e.value.code == ERR_CODE[case["error"]], str(e.value)
        if "message" in case:
            assert case["message"] in str(e.value)
        return
    got = [_dict_from_spec(l) for l in rg.load_inference_layers(path)]
    _same_layers(got, _expected(case), name)


@pytest.mark.parametrize("name", sorted(n for n, c in CASES.items() if c["canonical"]))
def test_product_writer_against_fixtures(rg, tmp_path, name):
    layers = [_spec_from_dict(d) for d in _expected(CASES[name])]
    p = tmp_path / "out.rtim"
    rg.save_layers(layers, p)
    assert p.read_bytes() == _fixture(name)


def test_product_and_oracle_write_the_same_bytes_for_exported_models(rg, tmp_path):
    """Exported models (every tag, every RTIM activation code) written by the
    product and by the oracle's restatement are the same bytes, and both read
    them back to the same layers."""
    from oracle import rtim
    for name, layers in _export_models(rg):
        p = tmp_path / f"{name}.rtim"
        rg.save_layers(layers, p)
        want = [_dict_from_spec(l) for l in layers]
        assert p.read_bytes() == rtim.save_layers(want), name
        _same_layers([_dict_from_spec(l) for l in rg.load_inference_layers(p)], want, name)
        _same_layers(rtim.load_layers(p.read_bytes()), want, name)


def test_loaded_sizes_outside_the_provider_are_refused_at_create(rg):
    """u32 sizes above 2^31 load unchanged (rtim_u32_fields), and creating a
    program from them is an RGNPU_ERR_INVALID error raised before any
    device work, like a ChannelAffine whose shift is shorter than its scale
    (the reference panics on both at compile or run time)."""
    layers = rg.load_inference_layers(os.path.join(GOLDEN, "rtim_u32_fields.rtim"))
    assert layers[0].in_features == 0x80000001 and layers[0].out_features == 0xFFFFFFFF
    assert layers[1].kernel == 0xFFFFFFFE and layers[1].stride == 0x80000000
    with pytest.raises(rg.RgnpuError) as e:
        rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    assert e.value.code == ERR_INVALID and "2^31" in str(e.value)
    short = [rg.LayerSpec.ChannelAffine(np.ones(3, np.float32), np.zeros(2, np.float32))]
    with pytest.raises(rg.RgnpuError) as e:
        rg.InferenceSession.from_layers(short, rg.ExecutionProvider.mi355x_int8())
    assert e.value.code == ERR_INVALID and "shorter" in str(e.value)


def _export_models(rg):
    """An MLP and a CNN whose exports hold tags 1-7 and activation codes 0-5
    (LeakyReLU with a slope), with BatchNorms that fold into their Linear or
    conv and one that stays a lone ChannelAffine (after a ReLU)."""
    from rustgears_amd import configs, nn
    from rustgears_amd.inference import Activation, LayerSpec
    rg.manual_seed(1103)
    bn1, bn2, bn3 = nn.BatchNorm1d(48), nn.BatchNorm1d(32), nn.BatchNorm2d(8)
    mlp = (nn.Sequential().add(nn.Linear(24, 48)).add(bn1).add(nn.LeakyRelu(0.0625))
           .add(nn.Linear(48, 40)).add(nn.Sigmoid()).add(nn.Linear(40, 40)).add(nn.Tanh())
           .add(nn.Linear(40, 32)).add(nn.Relu()).add(bn2)
           .add(nn.Linear(32, 32)).add(nn.Gelu()).add(nn.Linear(32, 12)))
    cnn = (nn.Sequential().add(nn.Conv2d(3, 8, 3).padding(1)).add(bn3).add(nn.Relu())
           .add(nn.MaxPool2d(2, 2)).add(nn.Conv2d(8, 16, 3).padding(1)).add(nn.Relu()).add(nn.MaxPool2d(2, 2))
           .add(nn.Flatten()).add(nn.Linear(16 * 4 * 4, 10)).add(nn.Softmax()))
    # running statistics as the quickstart draws them, so every BatchNorm
    # exports a non-trivial affine
    configs.set_bn_stats([bn1, bn2, bn3])
    mlp.eval()
    cnn.eval()
    mlp_layers = mlp.export() + [LayerSpec.Activation(Activation.NONE), LayerSpec.Softmax()]
    return [("mlp", mlp_layers), ("cnn", cnn.export())]


@pytest.mark.gpu
def test_saved_and_loaded_models_run_bit_exact_on_the_device(rg, ref, tmp_path):
    """save_layers -> load_inference_layers -> InferenceSession on the MI355X
    INT8 provider, every op's i8 activations, scales, i32 sums and f32
    outputs bit-exact with the oracle on the original layers."""
    inputs = {"mlp": lambda: rg.randn([96, 24]), "cnn": lambda: rg.randn([6, 3, 16, 16])}
    for name, layers in _export_models(rg):
        p = tmp_path / f"{name}.rtim"
        rg.save_layers(layers, p)
        loaded = rg.load_inference_layers(p)
        x = inputs[name]()
        print(f"[rtim] {name} x{tuple(x.shape)}", flush=True)
        sess = rg.InferenceSession.from_layers(loaded, rg.ExecutionProvider.mi355x_int8())
        y_plain = sess.run(x)
        sess.set_capture(True)
        y = sess.run(x)
        prog = ref.RefProgram(layers)
        prog.set_capture(True)
        yr = prog.run(x)
        assert sess.op_labels() == prog.labels(), name
        for i in range(prog.num_ops):
            for cap in (0, 1, 2, 3):
                want = prog.capture(i, cap)
                if want.size == 0 and cap != 3:
                    continue
                got = sess.capture(i, cap)
                tag = f"{name} op{i} ({prog.labels()[i]}) cap{cap}"
                if want.dtype == np.float32:
                    assert_bitexact_f32(got, want, tag)
                else:
                    assert np.array_equal(got, want), tag
        assert_bitexact_f32(y, yr, name + " output")
        assert_bitexact_f32(y_plain, yr, name + " output (production kernels)")
        prof = sess.last_npu_profile()
        assert prof.original_layers == prog.original_layers and prof.fused_ops == prog.num_ops
        assert prof.fp32_weight_bytes == prog.fp32_bytes and prof.npu_weight_bytes == prog.npu_bytes
        sess.close()
