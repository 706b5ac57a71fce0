"""GPU parity for special values that the fused GEMM paths never produce:
signed zeros through a standalone ReLU, and NaN / -inf / tie windows through
both max-pool kernels (the 2 x 2 stride-2 kernel and the general one).

Everything is compared bit for bit with the oracle, including the sign of
zero and the NaN payload a pool window keeps (kernels.rs:187: a later NaN
replaces an earlier one, equal values keep the first).
"""
import numpy as np
import pytest

from test_gpu_parity import check_against_oracle

pytestmark = pytest.mark.gpu

PRECISIONS = ("int8", "fp16", "fp32")


def _provider(rg, prec):
    return {"int8": rg.ExecutionProvider.mi355x_int8(), "fp16": rg.ExecutionProvider.mi355x_fp16(),
            "fp32": rg.ExecutionProvider.Gpu(0)}[prec]


def _ref_prec(ref, prec):
    return {"int8": ref.INT8, "fp16": ref.FP16, "fp32": ref.FP32}[prec]


def _run_bits(rg, ref, layers, x, prec, what):
    print(f"[special] {what} {prec} x{tuple(x.shape)}", flush=True)
    sess = rg.InferenceSession.from_layers(layers, _provider(rg, prec))
    y = sess.run(x)
    sess.close()
    want = ref.RefProgram(layers, precision=_ref_prec(ref, prec)).run(x)
    assert y.shape == want.shape, what
    yb, wb = y.view(np.uint32).reshape(-1), want.view(np.uint32).reshape(-1)
    if not np.array_equal(yb, wb):
        bad = np.flatnonzero(yb != wb)
        raise AssertionError(f"{what} {prec}: {bad.size} of {yb.size} differ, e.g. "
                             f"{[(int(i), hex(yb[i]), hex(wb[i])) for i in bad[:5]]}")
    return y


def _special_row():
    v = np.array([-0.0, 0.0, -1.5, 2.25, np.nan, -np.inf, np.inf, 1e-45, -1e-45, 3.0e38, -3.0e38, 1e-40],
                 np.float32)
    return v


@pytest.mark.parametrize("prec", PRECISIONS)
def test_standalone_relu_signed_zero(rg, ref, prec):
    """Activation(ReLU) alone: x.max(0.0) (backend.rs:71) gives +0.0 for
    -0.0 and for NaN, and keeps denormals (no flush to zero)."""
    from rustgears_amd.inference import Activation, LayerSpec
    x = np.tile(_special_row(), (7, 3)).astype(np.float32)
    y = _run_bits(rg, ref, [LayerSpec.Activation(Activation.RELU)], x, prec, "relu")
    assert y.view(np.uint32)[0, 0] == 0 and y.view(np.uint32)[0, 4] == 0
    # LeakyReLU keeps the sign of -0.0 (s * -0.0), NaN stays NaN
    _run_bits(rg, ref, [LayerSpec.Activation(Activation.leaky_relu(0.125))], x, prec, "leaky")


def test_relu_after_fp32_affine_signed_zero(rg, ref):
    """The FP32 provider keeps an unfolded ChannelAffine elementwise and runs
    ReLU as its own op (mod.rs:260-331): x * 1 + (-0.0) is -0.0 for x = -0.0,
    and the ReLU must turn it into +0.0."""
    from rustgears_amd.inference import Activation, LayerSpec
    c = 12
    layers = [LayerSpec.ChannelAffine(np.ones(c, np.float32), np.full(c, -0.0, np.float32)),
              LayerSpec.Activation(Activation.RELU)]
    x = np.tile(_special_row(), (5, 1)).astype(np.float32)
    pre = _run_bits(rg, ref, layers[:1], x, "fp32", "affine")
    assert pre.view(np.uint32)[0, 0] == 0x80000000
    y = _run_bits(rg, ref, layers, x, "fp32", "affine+relu")
    assert y.view(np.uint32)[0, 0] == 0


def _plant_pool_specials(x, nan_a, nan_b):
    """Windows of the 2 x 2, stride-2 grid in channel 0 of image 0 (and a few
    elsewhere): all NaN with two payloads, all -inf, signed-zero ties, a NaN
    after a larger value, +inf against NaN, equal finite values."""
    x[0, 0, 0:2, 0:2] = np.array([[nan_a, nan_b], [nan_a, nan_b]], np.float32)   # last NaN (payload b) wins
    x[0, 0, 2:4, 2:4] = -np.inf                                                   # stays -inf
    x[0, 0, 0:2, 2:4] = np.array([[-0.0, 0.0], [0.0, -0.0]], np.float32)         # first (-0.0) kept
    x[0, 0, 2:4, 0:2] = np.array([[0.0, -0.0], [-0.0, 0.0]], np.float32)         # first (+0.0) kept
    x[0, 1, 0:2, 0:2] = np.array([[9.0, 1.0], [nan_a, 3.0]], np.float32)         # NaN after 9 wins
    x[0, 1, 2:4, 2:4] = np.array([[np.inf, nan_b], [2.0, np.inf]], np.float32)   # NaN, then inf > NaN? no
    x[1, 2, 4:6, 4:6] = 7.5                                                       # ties of equal values
    x[2, 3, 0:2, 4:6] = np.array([[-np.inf, -np.inf], [-np.inf, -5.0]], np.float32)
    return x


@pytest.mark.parametrize("prec", PRECISIONS)
@pytest.mark.parametrize("k,s,h,w", [(2, 2, 8, 8), (2, 2, 8, 6), (3, 2, 9, 7), (2, 1, 6, 8)])
def test_maxpool_special_windows(rg, ref, prec, k, s, h, w):
    """MaxPool2d as the first layer, so its input holds the planted values
    (vision.rs:102-109, kernels.rs:180-191).  (2, 2, 8, 8) runs the 2 x 2
    stride-2 vector kernel; the others the general kernel."""
    from rustgears_amd.inference import LayerSpec
    nan_a = np.array([0x7fc00011], np.uint32).view(np.float32)[0]
    nan_b = np.array([0xffc00022], np.uint32).view(np.float32)[0]
    rg.manual_seed(31 + k * h + w)
    x = _plant_pool_specials(rg.randn([3, 4, h, w]), nan_a, nan_b)
    y = _run_bits(rg, ref, [LayerSpec.MaxPool2d(k, s)], x, prec, f"pool k{k} s{s} {h}x{w}")
    if k == 2 and s == 2:
        yb = y.view(np.uint32)
        assert yb[0, 0, 0, 0] == 0xffc00022 and np.isneginf(y[0, 0, 1, 1])
        assert yb[0, 0, 0, 1] == 0x80000000 and yb[0, 0, 1, 0] == 0


def test_maxpool_special_values_feed_quantized_consumers(rg, ref):
    """The INT8 pool also reduces the absmax its consumer quantizes with:
    per tensor for a Linear (NaN ignored like f32::max, quantized to 0) and
    per image for a Conv2d.  Checked op by op against the oracle's taps."""
    from rustgears_amd import nn
    from rustgears_amd.inference import LayerSpec
    nan_a = np.array([0x7fc00011], np.uint32).view(np.float32)[0]
    nan_b = np.array([0xffc00022], np.uint32).view(np.float32)[0]
    rg.manual_seed(77)
    x = _plant_pool_specials(rg.randn([3, 4, 8, 8]), nan_a, nan_b)
    x_finite = x.copy()
    x_finite[np.isinf(x_finite)] = 4.0
    rg.manual_seed(78)
    lin = [LayerSpec.MaxPool2d(2, 2), LayerSpec.Flatten()] + nn.Sequential().add(nn.Linear(64, 12)).export()
    check_against_oracle(rg, ref, lin, x_finite, "pool (NaN) -> linear")
    check_against_oracle(rg, ref, lin, x, "pool (NaN, inf) -> linear")
    conv = [LayerSpec.MaxPool2d(2, 2)] + nn.Sequential().add(nn.Conv2d(4, 8, 3)).add(nn.Relu()).export()
    check_against_oracle(rg, ref, conv, x_finite, "pool (NaN) -> conv")
