"""Conv -> MaxPool2d(2, 2) in the INT8 conv's epilogue (kernels.hip
conv_band_epilogue_pool2, program.cpp conv_pool_fusion).

Without capture the conv pools its own accumulator tile and stores only the
pool's output, raising the pool's absmax for the next op.  Capture turns the
fusion off, because capture keeps the conv's own output.  Each model's
output must equal both of these bit for bit:

* the oracle's output (npu.rs:319-390, the window rule of kernels.rs:180-191);
* the output with the fusion turned off (RGNPU_CONV_POOL=0).

The profile keeps the pool's record. A fused pool launches nothing.

Shapes the fusion does not take are checked too: width 24 or 64, odd height,
pool window 3, and sigmoid.  These run the conv and then the pool kernel.

The FP16 and FP32 direct convs (kernels.hip conv_direct_pool) pool the same
way.  FP32 convs carry no activation, so there the conv, its Act op and the
pool become one kernel.  Their fused output must equal the unfused one bit
for bit.  The unfused paths are checked against the oracle in
test_gpu_fp16.py and test_gpu_fp32.py.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def _run(rg, layers, x, fusion, fp16=False, fp32=False):
    import os
    os.environ["RGNPU_CONV_POOL"] = "1" if fusion else "0"
    try:
        if fp32:
            ep = rg.ExecutionProvider.Gpu(0)
        else:
            ep = rg.ExecutionProvider.mi355x_fp16() if fp16 else rg.ExecutionProvider.mi355x_int8()
        sess = rg.InferenceSession.from_layers(layers, ep)
        y = sess.run(x)
        y2 = sess.run(x)
        prof = sess.last_npu_profile()
        sess.close()
    finally:
        os.environ.pop("RGNPU_CONV_POOL", None)
    assert_bitexact_f32(y2, y, "second run")
    return y, prof


def _check(rg, ref, layers, x, what, fused_pools):
    print(f"[conv-pool] {what} x{tuple(x.shape)}", flush=True)
    want = ref.RefProgram(layers).run(x, parallel=True)
    y, prof = _run(rg, layers, x, True)
    assert_bitexact_f32(y, want, f"{what} (fused)")
    y0, prof0 = _run(rg, layers, x, False)
    assert_bitexact_f32(y0, want, f"{what} (unfused)")
    pools = [r for r in prof.records if r.op.startswith("NPU::MaxPool2d")]
    pools0 = [r for r in prof0.records if r.op.startswith("NPU::MaxPool2d")]
    assert [r.op for r in prof.records] == [r.op for r in prof0.records]
    assert [r.kernel_ns == 0 for r in pools] == fused_pools, (what, pools)
    assert all(r.kernel_ns > 0 for r in pools0), (what, pools0)


def test_cnn_bench_config(rg, ref):
    from rustgears_amd import configs
    model, x = configs.cnn()
    _check(rg, ref, model.export(), x, "cnn[256,3,32,32]", [True, True])


def _conv_pool_model(rg, seed, c, o, hw, act, tail, pool_k=2):
    from rustgears_amd import nn
    rg.manual_seed(seed)
    m = nn.Sequential().add(nn.Conv2d(c, o, 3).padding(1))
    if act == "relu":
        m.add(nn.Relu())
    elif act == "sigmoid":
        m.add(nn.Sigmoid())
    m.add(nn.MaxPool2d(pool_k))
    if tail == "linear":
        oh, ow = hw[0] // pool_k, hw[1] // pool_k
        m.add(nn.Flatten()).add(nn.Linear(o * oh * ow, 7))
    elif tail == "conv":
        m.add(nn.Conv2d(o, 8, 3).padding(1)).add(nn.Relu())
    return m.export()


CASES = [
    # (name, c, o, (h, w), act, tail, images, fused)
    ("width 32, linear after", 3, 32, (32, 32), "relu", "linear", 6, True),
    ("width 16, conv after", 8, 64, (16, 16), "relu", "conv", 5, True),
    ("no activation, pool is the output", 4, 32, (16, 32), None, None, 3, True),
    ("128-pixel tiles (wide weights)", 320, 32, (16, 16), "relu", "linear", 3, True),
    ("odd channel count, ragged O", 5, 40, (32, 16), "relu", "conv", 2, True),
    ("width 24: not fused", 3, 32, (24, 24), "relu", "linear", 2, False),
    ("width 64: not fused", 3, 32, (8, 64), "relu", "linear", 2, False),
    ("odd height: not fused", 3, 32, (15, 16), "relu", "linear", 2, False),
    ("sigmoid: not fused", 3, 32, (16, 16), "sigmoid", "linear", 2, False),
]


@pytest.mark.parametrize("name,c,o,hw,act,tail,n,fused", CASES, ids=[c[0] for c in CASES])
def test_conv_pool_shapes(rg, ref, name, c, o, hw, act, tail, n, fused):
    layers = _conv_pool_model(rg, 300 + c + o, c, o, hw, act, tail)
    x = rg.randn([n, c, hw[0], hw[1]])
    _check(rg, ref, layers, x, name, [fused])


def test_pool_window_3_is_not_fused(rg, ref):
    layers = _conv_pool_model(rg, 41, 3, 32, (16, 16), "relu", "linear", pool_k=3)
    x = rg.randn([2, 3, 16, 16])
    _check(rg, ref, layers, x, "pool 3", [False])


@pytest.mark.parametrize("act", ["relu", None], ids=["relu", "no-activation"])
def test_special_values_through_the_fused_pool(rg, ref, act):
    """NaN and -inf bias channels: the window rule keeps a NaN and an all
    -inf window gives -inf (no activation), ReLU turns both into values it
    defines; a channel of large negative bias gives windows of equal values
    (ReLU zeros), where the first element is kept."""
    layers = _conv_pool_model(rg, 77, 4, 32, (16, 32), act, None)
    conv = layers[0]
    conv.bias[[1, 9]] = np.float32(np.nan)
    conv.bias[[4, 20]] = np.float32(-np.inf)
    conv.bias[[6]] = np.float32(-1e3)
    x = rg.randn([3, 4, 16, 32])
    _check(rg, ref, layers, x, f"special values, act {act}", [True])


def test_capture_turns_the_fusion_off(rg, ref):
    """A capture run keeps the conv's own output; switching capture on and
    off on one session rebuilds the plan each time."""
    from rustgears_amd import configs
    model, x = configs.cnn(n=8)
    layers = model.export()
    want = ref.RefProgram(layers).run(x, parallel=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    assert_bitexact_f32(y, want, "fused")
    assert [r.kernel_ns == 0 for r in sess.last_npu_profile().records if "MaxPool" in r.op] == [True, True]
    sess.set_capture(True)
    y = sess.run(x)
    assert_bitexact_f32(y, want, "capture")
    p = ref.RefProgram(layers)
    p.set_capture(True)
    p.run(x, parallel=True)
    assert_bitexact_f32(sess.capture(0, 3), p.capture(0, 3), "conv 1 output (capture)")
    assert all(r.kernel_ns > 0 for r in sess.last_npu_profile().records if "MaxPool" in r.op)
    sess.set_capture(False)
    y = sess.run(x)
    assert_bitexact_f32(y, want, "fused again")
    assert [r.kernel_ns == 0 for r in sess.last_npu_profile().records if "MaxPool" in r.op] == [True, True]
    sess.close()


FP16_CASES = [
    # (name, c, o, (h, w), act, tail, images, fused)
    ("bench CNN's first conv", 3, 32, (32, 32), "relu", "conv", 4, True),
    ("width 16, 64 channels, no activation", 3, 64, (16, 16), None, "linear", 3, True),
    ("ragged last wave (L = 16 x 6)", 2, 16, (6, 16), "relu", None, 5, True),
    ("odd height: not fused", 3, 32, (15, 16), "relu", "linear", 2, False),
    ("width 64: not fused", 3, 32, (8, 64), "relu", "linear", 2, False),
]


@pytest.mark.parametrize("name,c,o,hw,act,tail,n,fused", FP16_CASES, ids=[c[0] for c in FP16_CASES])
def test_fp16_direct_conv_pool(rg, name, c, o, hw, act, tail, n, fused):
    layers = _conv_pool_model(rg, 500 + c + o, c, o, hw, act, tail)
    x = rg.randn([n, c, hw[0], hw[1]])
    print(f"[conv-pool fp16] {name} x{tuple(x.shape)}", flush=True)
    y, prof = _run(rg, layers, x, True, fp16=True)
    y0, prof0 = _run(rg, layers, x, False, fp16=True)
    assert_bitexact_f32(y, y0, name)
    pools = [r for r in prof.records if r.op.startswith("NPU::MaxPool2d")]
    assert [r.kernel_ns == 0 for r in pools][:1] == [fused], (name, pools)
    assert all(r.kernel_ns > 0 for r in prof0.records if r.op.startswith("NPU::MaxPool2d"))


def test_fp16_special_values_through_the_fused_pool(rg):
    layers = _conv_pool_model(rg, 91, 3, 32, (16, 32), None, None)
    conv = layers[0]
    conv.bias[[1, 9]] = np.float32(np.nan)
    conv.bias[[4, 20]] = np.float32(-np.inf)
    x = rg.randn([3, 3, 16, 32])
    y, _ = _run(rg, layers, x, True, fp16=True)
    y0, _ = _run(rg, layers, x, False, fp16=True)
    assert_bitexact_f32(y, y0, "fp16 special values")


FP32_CASES = [
    # (name, c, o, (h, w), act, tail, images, fused)
    ("conv, ReLU, pool (bench CNN's first conv)", 3, 32, (32, 32), "relu", "conv", 4, True),
    ("conv, pool: no Act op between", 3, 64, (16, 16), None, "linear", 3, False),
    ("ragged last wave", 2, 16, (6, 16), "relu", None, 5, True),
    ("sigmoid: not fused", 3, 32, (16, 16), "sigmoid", "linear", 2, False),
]


@pytest.mark.parametrize("name,c,o,hw,act,tail,n,fused", FP32_CASES, ids=[c[0] for c in FP32_CASES])
def test_fp32_direct_conv_act_pool(rg, name, c, o, hw, act, tail, n, fused):
    layers = _conv_pool_model(rg, 700 + c + o, c, o, hw, act, tail)
    x = rg.randn([n, c, hw[0], hw[1]])
    print(f"[conv-pool fp32] {name} x{tuple(x.shape)}", flush=True)
    y, prof = _run(rg, layers, x, True, fp32=True)
    y0, prof0 = _run(rg, layers, x, False, fp32=True)
    assert_bitexact_f32(y, y0, name)
    if prof is not None and prof.records:
        pools = [r for r in prof.records if "MaxPool2d" in r.op]
        assert [r.kernel_ns == 0 for r in pools][:1] == [fused], (name, pools)
