"""The inputs of the M <= 8 GEMV (QuantTensor::from_f32, quantize.rs:18-24,
at npu.rs:312, then quantize.rs:93-118 with the rows streamed once).

Bit for bit against the oracle, capture taps included:

* every M from 1 to 8, with the scale from the input's own absmax (the
  run's first Linear: the one-pass input quantization, a single workgroup
  at these sizes) and from the producer's absmax slot (a GEMV after a GEMV);
* inputs holding NaN, +-inf and the absmax at the last column;
* K % 4 != 0 (element loads), a long K (the input larger than one
  workgroup keeps), and an input pointer that is not 16-byte aligned
  (run_device on an offset buffer);
* the matrix-core form (M >= 2, K a multiple of 512, at least 4096 output
  rows): 512-byte K pieces that do not split evenly over a workgroup's 4
  waves, N not a multiple of 16, a grid of more workgroups than CUs (more
  than 8 row blocks per CU), and a GEMV after a GEMV;
* the one-row form that quantizes its own f32 input: with the input's own
  absmax (the run's first Linear) and with the producer's, K at the largest
  row it stages (8192) and just past it, K % 4 != 0 and an unaligned input
  (both take the separate quantize pass);
* one-row GEMVs after a one-row GEMV whose rows are past that staging (the
  producer's absmax, a separate quantize pass), without capture: a ragged K,
  the G layer-2 shape, K % 4 != 0, and NaN and +-inf in the input.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32
from test_gpu_parity import check_against_oracle

pytestmark = pytest.mark.gpu


def _mlp(rg, dims, seed, act="gelu"):
    from rustgears_amd import nn
    rg.manual_seed(seed)
    acts = {"tanh": nn.Tanh, "relu": nn.Relu, "gelu": nn.Gelu}
    m = nn.Sequential()
    for i, (a, b) in enumerate(zip(dims[:-1], dims[1:])):
        m.add(nn.Linear(a, b))
        if i + 2 < len(dims):
            m.add(acts[act]())
    return m.export()


@pytest.mark.parametrize("rows", list(range(1, 9)))
def test_gemv_every_m(rg, ref, rows):
    layers = _mlp(rg, [1000, 3000, 700], seed=50 + rows)
    x = rg.randn([rows, 1000])
    check_against_oracle(rg, ref, layers, x, f"gemv M={rows}")
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    sess.close()
    assert_bitexact_f32(y, ref.RefProgram(layers).run(x), f"gemv M={rows} (no capture)")


def test_gemv_special_values(rg, ref):
    layers = _mlp(rg, [512, 1024, 64], seed=7, act="relu")
    x = rg.randn([4, 512])
    x[0, 3] = np.nan
    x[1, 511] = -1234.5  # the absmax, at the last column
    check_against_oracle(rg, ref, layers, x, "gemv NaN / absmax last column")
    x2 = x.copy()
    x2[2, 100] = np.inf
    x2[3, 7] = -np.inf
    check_against_oracle(rg, ref, layers, x2, "gemv inf")


@pytest.mark.parametrize("dims,rows", [([333, 600, 40], 3), ([20000, 1024, 64], 8)], ids=["K%4", "long K"])
def test_gemv_odd_and_long_rows(rg, ref, dims, rows):
    layers = _mlp(rg, dims, seed=rows + dims[0])
    check_against_oracle(rg, ref, layers, rg.randn([rows, dims[0]]), f"gemv {dims} M={rows}")


def test_unaligned_device_input(rg, ref):
    from rustgears_amd.inference import DeviceBuffer
    layers = _mlp(rg, [1024, 2048, 256], seed=3)
    x = rg.randn([2, 1024])
    want = ref.RefProgram(layers).run(x)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    buf = DeviceBuffer(x.nbytes + 16)
    padded = np.zeros(x.size + 4, np.float32)
    padded[1:1 + x.size] = x.reshape(-1)
    buf.upload(padded)

    class Offset:  # the same allocation, 4 bytes in
        ptr = buf.ptr + 4
        nbytes = x.nbytes

    d_y = DeviceBuffer(2 * 256 * 4)
    for src, what in ((Offset, "unaligned"),):
        assert sess.run_device(src, x.shape, d_y) == (2, 256)
        sess.synchronize()
        assert_bitexact_f32(d_y.download((2, 256)), want, f"gemv {what} input")
    d_x = DeviceBuffer.from_array(x)
    sess.run_device(d_x, x.shape, d_y)
    sess.synchronize()
    assert_bitexact_f32(d_y.download((2, 256)), want, "gemv aligned input")
    sess.close()


MFMA_CASES = [
    # (dims, rows): 2560 = 5 K pieces over 4 waves; 4100 outputs -> 272 row
    # blocks, the last one partly padding; 33000 -> 2064 blocks, 258
    # workgroups of at most 8; [.., 4096, 4608] a GEMV feeding a GEMV
    ([2560, 4100, 64], 2),
    ([2560, 4100, 64], 5),
    ([2560, 4100, 64], 8),
    ([2048, 33000, 16], 3),
    ([3072, 4096, 4608, 40], 7),
]


@pytest.mark.parametrize("dims,rows", MFMA_CASES, ids=[f"{c[0][1]}-M{c[1]}" for c in MFMA_CASES])
def test_gemv_matrix_core_form(rg, ref, dims, rows):
    layers = _mlp(rg, dims, seed=rows * 7 + dims[1], act="tanh")
    x = rg.randn([rows, dims[0]])
    check_against_oracle(rg, ref, layers, x, f"gemv mfma {dims} M={rows}")
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    y2 = sess.run(x)
    sess.close()
    want = ref.RefProgram(layers).run(x)
    assert_bitexact_f32(y, want, f"gemv mfma {dims} M={rows} (no capture)")
    assert_bitexact_f32(y2, want, f"gemv mfma {dims} M={rows} (second run)")


XQ_CASES = [
    # (dims, what)
    ([8192, 4096, 8192, 24], "largest staged row, twice"),
    ([8196, 1024, 512], "row past the staged limit"),
    ([1022, 2048, 4100, 64], "K % 4 != 0 first, then staged"),
    ([4000, 28672, 8192], "staged, then a row past the limit"),
]


@pytest.mark.parametrize("dims,what", XQ_CASES, ids=[c[1] for c in XQ_CASES])
def test_gemv_one_row_quantizing_its_input(rg, ref, dims, what):
    layers = _mlp(rg, dims, seed=dims[0] + len(dims), act="gelu")
    x = rg.randn([1, dims[0]])
    x[0, dims[0] - 1] = 17.75  # the absmax at the last column
    check_against_oracle(rg, ref, layers, x, f"gemv xq {what}")
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    y2 = sess.run(x)
    sess.close()
    want = ref.RefProgram(layers).run(x)
    assert_bitexact_f32(y, want, f"gemv xq {what} (no capture)")
    assert_bitexact_f32(y2, want, f"gemv xq {what} (second run)")


def test_gemv_one_row_unaligned_input(rg, ref):
    from rustgears_amd.inference import DeviceBuffer
    layers = _mlp(rg, [2048, 4096, 300], seed=11)
    x = rg.randn([1, 2048])
    want = ref.RefProgram(layers).run(x)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    buf = DeviceBuffer(x.nbytes + 16)
    padded = np.zeros(x.size + 4, np.float32)
    padded[1:1 + x.size] = x.reshape(-1)
    buf.upload(padded)

    class Offset:  # the same allocation, 4 bytes in
        ptr = buf.ptr + 4
        nbytes = x.nbytes

    d_y = DeviceBuffer(300 * 4)
    assert sess.run_device(Offset, x.shape, d_y) == (1, 300)
    sess.synchronize()
    assert_bitexact_f32(d_y.download((1, 300)), want, "gemv one row, unaligned input")
    d_x = DeviceBuffer.from_array(x)
    sess.run_device(d_x, x.shape, d_y)
    sess.synchronize()
    assert_bitexact_f32(d_y.download((1, 300)), want, "gemv one row, aligned input")
    sess.close()


LONG_ROW_CASES = [
    # (dims, what): the second layer's row is longer than gemv_xq stages
    ([1000, 9004, 100], "ragged K past the staged row"),
    ([3000, 28672, 4096], "G layer-2 shape"),
    ([1000, 8198, 64], "K % 4 != 0"),
]


@pytest.mark.parametrize("dims,what", LONG_ROW_CASES, ids=[c[1] for c in LONG_ROW_CASES])
def test_gemv_one_row_after_a_long_row(rg, ref, dims, what):
    layers = _mlp(rg, dims, seed=dims[1] + 3, act="gelu")
    x = rg.randn([1, dims[0]])
    want = ref.RefProgram(layers).run(x)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    y2 = sess.run(x)
    recs = sess.last_npu_profile().records
    sess.close()
    assert_bitexact_f32(y, want, f"gemv long row {what}")
    assert_bitexact_f32(y2, want, f"gemv long row {what} (second run)")
    assert recs[1].kernel_ns > 0, recs[1]
    check_against_oracle(rg, ref, layers, x, f"gemv long row {what} (capture)")


def test_gemv_long_row_special_values(rg, ref):
    """NaN and +-inf in the long row the second GEMV reads (planted through
    the first layer's bias): the absmax is +inf, so the scale is +inf and
    every value quantizes to 0 (NaN * 0 and inf * 0 are NaN, which quantize
    to 0 as well); then a NaN-only column with finite others."""
    for what, plant in (("inf and NaN", {5: np.nan, 9: np.inf, 12: -np.inf}), ("NaN only", {5: np.nan})):
        layers = _mlp(rg, [512, 9000, 64], seed=3, act="gelu")  # GELU keeps NaN and +inf (-inf becomes NaN)
        for col, v in plant.items():
            layers[0].bias[col] = v
        x = rg.randn([1, 512])
        want = ref.RefProgram(layers).run(x)
        sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
        y = sess.run(x)
        sess.close()
        assert_bitexact_f32(y, want, f"gemv long row {what}")
