"""Loader for the committed golden fixtures in tests/golden/ (written by
tests/golden/make_golden.py from the oracle).  Each case is a JSON layer
list plus an .npz of arrays: inputs, outputs and per-op captures."""
import json
import os

import numpy as np

from rustgears_amd.inference import Activation, LayerSpec

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
CAP_NAMES = {"qact": 0, "scale": 1, "acc": 2, "out": 3}


def layers_from_json(desc, arrays):
    out = []
    for d in desc:
        k = d["kind"]
        if k == "Linear":
            out.append(LayerSpec.Linear(d["in"], d["out"], arrays[d["weight"]], arrays[d["bias"]]))
        elif k == "Conv2d":
            out.append(LayerSpec.Conv2d(d["in"], d["out"], d["k"], d["s"], d["p"], arrays[d["weight"]],
                                        arrays[d["bias"]]))
        elif k == "ChannelAffine":
            out.append(LayerSpec.ChannelAffine(arrays[d["scale"]], arrays[d["shift"]]))
        elif k == "MaxPool2d":
            out.append(LayerSpec.MaxPool2d(d["k"], d["s"]))
        elif k == "Flatten":
            out.append(LayerSpec.Flatten())
        elif k == "Activation":
            out.append(LayerSpec.Activation(Activation(d["code"], d.get("param", 0.0))))
        elif k == "Softmax":
            out.append(LayerSpec.Softmax())
    return out


def load(name):
    with open(os.path.join(GOLDEN, name + ".json")) as f:
        meta = json.load(f)
    arrays = dict(np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False))
    caps = []
    for i in range(meta["num_ops"]):
        c = {}
        for cname, code in CAP_NAMES.items():
            key = f"op{i}_{cname}"
            if key in arrays:
                c[code] = arrays[key]
        caps.append(c)
    return {"name": name, "layers": layers_from_json(meta["layers"], arrays), "x": arrays["x"],
            "y": arrays["y"], "caps": caps, "labels": meta["labels"], "fp32_bytes": meta["fp32_bytes"],
            "npu_bytes": meta["npu_bytes"]}


def names():
    # a model case is a .json layer list with its .npz arrays (the RTIM byte
    # fixtures' rtim_cases.json has none)
    return sorted(f[:-5] for f in os.listdir(GOLDEN)
                  if f.endswith(".json") and os.path.exists(os.path.join(GOLDEN, f[:-5] + ".npz")))


def load_all():
    return [load(n) for n in names()]
