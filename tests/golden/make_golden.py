"""Writes the golden fixtures in this directory from the CPU oracle.

Cases are ReLU / LeakyReLU / None only, so their values do not depend on the
host libm.  Run from the repo root:  python tests/golden/make_golden.py
Each case: <name>.json (layer list, labels, byte counts) and <name>.npz
(weights, input x, output y, and per-op captures op<i>_{qact,scale,acc,out}).
"""
import json
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)

import oracle  # noqa: E402
import rustgears_amd as rg  # noqa: E402
from rustgears_amd import configs, nn  # noqa: E402
from rustgears_amd.inference import Activation, LayerSpec  # noqa: E402


def describe(layers, arrays):
    desc = []
    for i, l in enumerate(layers):
        t = type(l).__name__
        if t == "Linear":
            arrays[f"w{i}"], arrays[f"b{i}"] = l.weight, l.bias
            desc.append({"kind": t, "in": l.in_features, "out": l.out_features, "weight": f"w{i}", "bias": f"b{i}"})
        elif t == "Conv2d":
            arrays[f"w{i}"], arrays[f"b{i}"] = l.weight, l.bias
            desc.append({"kind": t, "in": l.in_channels, "out": l.out_channels, "k": l.kernel, "s": l.stride,
                         "p": l.padding, "weight": f"w{i}", "bias": f"b{i}"})
        elif t == "ChannelAffine":
            arrays[f"sc{i}"], arrays[f"sh{i}"] = l.scale, l.shift
            desc.append({"kind": t, "scale": f"sc{i}", "shift": f"sh{i}"})
        elif t == "MaxPool2d":
            desc.append({"kind": t, "k": l.kernel, "s": l.stride})
        elif t == "Activation":
            desc.append({"kind": t, "code": l.act.code, "param": l.act.param})
        else:
            desc.append({"kind": t})
    return desc


def write(name, layers, x):
    arrays = {"x": np.ascontiguousarray(x, np.float32)}
    desc = describe(layers, arrays)
    p = oracle.RefProgram(layers)
    p.set_capture(True)
    arrays["y"] = p.run(x)
    for i in range(p.num_ops):
        for cname, code in (("qact", 0), ("scale", 1), ("acc", 2), ("out", 3)):
            c = p.capture(i, code)
            if c.size:
                arrays[f"op{i}_{cname}"] = c
    meta = {"layers": desc, "labels": p.labels(), "num_ops": p.num_ops, "fp32_bytes": p.fp32_bytes,
            "npu_bytes": p.npu_bytes, "input_shape": list(x.shape), "output_shape": list(arrays["y"].shape)}
    with open(os.path.join(HERE, name + ".json"), "w") as f:
        json.dump(meta, f, indent=1)
    np.savez_compressed(os.path.join(HERE, name + ".npz"), **arrays)
    print(name, p.labels(), arrays["y"].shape)


def main():
    # 1. the quickstart MLP (configs.quickstart, the 4 -> 32 -> 3 example of the reference's USAGE.md)
    model, x = configs.quickstart()
    write("quickstart_mlp", model.export(), x)

    # 2. tiny CNN: padding, stride 2, partial coverage (k=2, s=3), pooling,
    #    LeakyReLU, flatten into Linear
    rg.manual_seed(11)
    c1, bn = nn.Conv2d(2, 5, 3).padding(1), nn.BatchNorm2d(5)
    c2 = nn.Conv2d(5, 4, 2).stride(3)
    l1, l2 = nn.Linear(4 * 2 * 2, 6), nn.Linear(6, 3)
    configs.set_bn_stats([bn])
    model = (nn.Sequential().add(c1).add(bn).add(nn.Relu()).add(nn.MaxPool2d(2)).add(c2).add(nn.Relu())
             .add(nn.Flatten()).add(l1).add(nn.LeakyRelu(0.1)).add(l2))
    x = rg.randn([3, 2, 12, 12])
    write("tiny_cnn", model.export(), x)

    # 3. quantization edge cases: NaN in the input, an all-zero row, lone
    #    ChannelAffine (diagonal GEMM), standalone ReLU, ragged K and N
    rng = np.random.default_rng(7)
    x = rng.standard_normal((5, 37)).astype(np.float32)
    x[0, 3] = np.nan
    x[2, :] = 0.0
    w1 = rng.standard_normal(37 * 19).astype(np.float32) * 0.2
    b1 = rng.standard_normal(19).astype(np.float32)
    layers = [LayerSpec.Linear(37, 19, w1, b1), LayerSpec.ChannelAffine(np.linspace(0.5, 1.5, 19).astype(np.float32),
                                                                        np.linspace(-1, 1, 19).astype(np.float32)),
              LayerSpec.Activation(Activation.RELU),
              LayerSpec.ChannelAffine(np.linspace(2, -2, 19).astype(np.float32), np.zeros(19, np.float32)),
              LayerSpec.Activation(Activation.RELU)]
    write("quant_edges", layers, x)


if __name__ == "__main__":
    main()
