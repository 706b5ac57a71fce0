"""Two INT8 conv + MaxPool2d(2, 2) stages as one kernel per image
(kernels.hip conv_pool_pair_kernel, program.cpp make_plan).

Conv A (at most 4 channels -> 32, 3 x 3, stride 1, pad 1, on 32 x 32 images,
the run's first op) then conv B (32 -> 64, the same window), each with ReLU
or no activation and followed by its pool: one workgroup per image keeps the
pooled conv A output in LDS and quantizes it for conv B with that image's
own scale (npu.rs:341-351), as the two convs do.  Each model's output must
equal bit for bit the oracle's and the output with the pair turned off
(RGNPU_CONV_PAIR=0: the two conv + pool kernels): the CNN benchmark config,
1 to 7 images, 1 to 4 input channels, every activation combination, and
NaN, infinities and an all-zero image.  Programs the kernel does not take
(28 x 28 images, 48 channels after conv B, a second conv that is not pooled)
run the separate convs.  The profile keeps every op's record; conv B's
reports 0 ns when the pair runs.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def _model(rg, seed, c, hw=32, acts=("relu", "relu"), ob=64, pool_b=True, bn=True):
    from rustgears_amd import configs, nn
    rg.manual_seed(seed)
    m, bns = nn.Sequential(), []
    mods = {"relu": nn.Relu, None: None}
    for i, (cin, cout) in enumerate(((c, 32), (32, ob))):
        m.add(nn.Conv2d(cin, cout, 3).padding(1))
        if bn:
            b = nn.BatchNorm2d(cout)
            bns.append(b)
            m.add(b)
        if acts[i]:
            m.add(mods[acts[i]]())
        if i == 0 or pool_b:
            m.add(nn.MaxPool2d(2))
    side = hw // 4 if pool_b else hw // 2
    m.add(nn.Flatten()).add(nn.Linear(ob * side * side, 10))
    configs.set_bn_stats(bns)
    return m.export()


def _run(rg, layers, x, pair, monkeypatch):
    if pair:
        monkeypatch.delenv("RGNPU_CONV_PAIR", raising=False)
    else:
        monkeypatch.setenv("RGNPU_CONV_PAIR", "0")
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    y2 = sess.run(x)
    recs = list(sess.last_npu_profile().records)
    sess.close()
    monkeypatch.delenv("RGNPU_CONV_PAIR", raising=False)
    assert_bitexact_f32(y2, y, "second run")
    return y, recs


def _check(rg, ref, monkeypatch, layers, x, what, expect_pair=True):
    print(f"[conv-pair] {what} x{tuple(x.shape)}", flush=True)
    want = ref.RefProgram(layers).run(x, parallel=True)
    y, recs = _run(rg, layers, x, True, monkeypatch)
    y0, recs0 = _run(rg, layers, x, False, monkeypatch)
    assert_bitexact_f32(y, want, f"{what} (pair) vs oracle")
    assert_bitexact_f32(y0, want, f"{what} (separate convs) vs oracle")
    assert [r.op for r in recs] == [r.op for r in recs0]
    convs = [r for r in recs if r.op.startswith("NPU::FusedConv2dAct") or r.op.startswith("NPU::Conv2d")]
    convs0 = [r for r in recs0 if r.op.startswith("NPU::FusedConv2dAct") or r.op.startswith("NPU::Conv2d")]
    assert convs[0].kernel_ns > 0 and all(r.kernel_ns > 0 for r in convs0), (convs, convs0)
    assert (convs[1].kernel_ns == 0 and convs[1].duration_ns == 0) == expect_pair, convs


def test_cnn_bench_config(rg, ref, monkeypatch):
    from rustgears_amd import configs
    model, x = configs.cnn()
    _check(rg, ref, monkeypatch, model.export(), x, "cnn[256,3,32,32]")


CASES = [
    # (n, c, acts, bn)
    (1, 3, ("relu", "relu"), True),
    (7, 1, (None, "relu"), True),
    (5, 4, ("relu", None), False),
    (3, 2, (None, None), True),
]


@pytest.mark.parametrize("n,c,acts,bn", CASES, ids=[f"n{n}-c{c}-{a[0]}-{a[1]}" for n, c, a, _ in CASES])
def test_pair_shapes_and_activations(rg, ref, monkeypatch, n, c, acts, bn):
    layers = _model(rg, seed=40 + n * 4 + c, c=c, acts=acts, bn=bn)
    x = rg.randn([n, c, 32, 32]) * np.float32(2.0)
    _check(rg, ref, monkeypatch, layers, x, f"pair n={n} c={c} {acts}")


def test_pair_special_values(rg, ref, monkeypatch):
    """NaN is ignored by each image's absmax and quantizes to 0; an infinite
    pixel makes its image's scale infinite (every value quantizes to 0, the
    conv A sums are 0 and their products with the infinite scale NaN); an
    all-zero image has scale 1.  Each image is quantized on its own."""
    layers = _model(rg, seed=9, c=3, acts=(None, "relu"))
    x = rg.randn([4, 3, 32, 32])
    x[0, 1, 5, 7] = np.nan
    x[0, 2, 31, 0] = -np.nan
    x[1, 0, 0, 0] = np.inf
    x[2] = 0.0
    x[3, 0, 16, 16] = -3e38
    _check(rg, ref, monkeypatch, layers, x, "pair special values")


NOT_TAKEN = [
    # (what, kwargs): the separate conv + pool kernels run
    ("28x28 images", dict(hw=28)),
    ("48 channels after conv B", dict(ob=48)),
    ("conv B not pooled", dict(pool_b=False)),
]


@pytest.mark.parametrize("what,kw", NOT_TAKEN, ids=[w for w, _ in NOT_TAKEN])
def test_programs_the_pair_does_not_take(rg, ref, monkeypatch, what, kw):
    hw = kw.get("hw", 32)
    layers = _model(rg, seed=13, c=3, **kw)
    _check(rg, ref, monkeypatch, layers, rg.randn([3, 3, hw, hw]), what, expect_pair=False)
