"""rgnpu_program_run_device_noalloc: the allocation-free variant of
rgnpu_program_run_device, whose intermediate buffers live in the library's
per-device scratch array instead of allocations of their own.

Through the C ABI, against rgnpu_program_run_device on the same program and
input, bit for bit, on two calls in a row, the second with a smaller input;
another program's allocation-free call between them leaves different data
in the shared scratch.  Covered: INT8 Linear chains with the fused
requantization (two i8 operand buffers, barrier words in the slots), a
Linear on the small-tile GEMM whose K slices meet in sum words of the slot
set, an INT8
conv net with partial window coverage (masks uploaded by every call), FP16
convs with split K (workspace and the [n*L, O] staging buffer) and the FP32
provider.  A shape whose buffers exceed the scratch is refused with
RGNPU_ERR_CAPACITY before anything is enqueued, and the next call works.
"""
import ctypes

import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu

ERR_CAPACITY = 7


def _noalloc(sess, d_x, shape, d_y):
    from rustgears_amd import _native as N
    sh = (ctypes.c_int64 * len(shape))(*shape)
    shp = (ctypes.c_int64 * 8)()
    nd = ctypes.c_int32()
    st = N.lib().rgnpu_program_run_device_noalloc(sess._h, d_x.ptr if d_x else None, sh, len(shape),
                                                 d_y.ptr if d_y else None, d_y.nbytes // 4 if d_y else 0, shp,
                                                 ctypes.byref(nd))
    return st, tuple(shp[i] for i in range(nd.value))


def _both(rg, sess, x, what):
    """(run_device output, run_device_noalloc output) for input x."""
    from rustgears_amd.inference import DeviceBuffer
    print(f"[noalloc] {what} x{tuple(x.shape)}", flush=True)
    d_x = DeviceBuffer.from_array(x)
    st, shp = _noalloc(sess, d_x, x.shape, None)  # shape query: nothing enqueued
    assert st == 0, st
    n = int(np.prod(shp))
    d_ref, d_na = DeviceBuffer(max(n, 1) * 4), DeviceBuffer(max(n, 1) * 4)
    assert sess.run_device(d_x, x.shape, d_ref) == shp
    st, shp2 = _noalloc(sess, d_x, x.shape, d_na)
    assert st == 0 and shp2 == shp
    sess.synchronize()
    return d_ref.download(shp), d_na.download(shp)


def _mlp(rg, dims, act, seed):
    from rustgears_amd import nn
    rg.manual_seed(seed)
    m = nn.Sequential()
    for a, b in zip(dims[:-1], dims[1:]):
        m.add(nn.Linear(a, b)).add(act())
    return m.export()


def _cnn(rg, seed, stride):
    from rustgears_amd import nn
    rg.manual_seed(seed)
    m = (nn.Sequential().add(nn.Conv2d(3, 16, 3).stride(stride)).add(nn.Relu())
         .add(nn.Conv2d(16, 32, 3).padding(1)).add(nn.Relu()).add(nn.MaxPool2d(2)).add(nn.Flatten()))
    return m


def _providers(rg):
    return {"int8": rg.ExecutionProvider.mi355x_int8(), "fp16": rg.ExecutionProvider.mi355x_fp16(),
            "fp32": rg.ExecutionProvider.Gpu(0)}


@pytest.mark.parametrize("prec", ["int8", "fp16", "fp32"])
def test_noalloc_matches_run_device_mlp(rg, ref, prec):
    from rustgears_amd import nn
    layers = _mlp(rg, [256, 384, 512, 384, 130], nn.Tanh, seed=5)
    other = _mlp(rg, [96, 200, 64], nn.Gelu, seed=6)
    sess = rg.InferenceSession.from_layers(layers, _providers(rg)[prec])
    sess2 = rg.InferenceSession.from_layers(other, _providers(rg)[prec])
    x1, x2, xo = rg.randn([300, 256]), rg.randn([40, 256]), rg.randn([700, 96])
    a, b = _both(rg, sess, x1, f"mlp {prec} 300 rows")
    assert_bitexact_f32(b, a, f"mlp {prec} 300 rows")
    if prec == "int8":
        assert_bitexact_f32(b, ref.RefProgram(layers).run(x1, parallel=True), "mlp int8 vs oracle")
    c, d = _both(rg, sess2, xo, f"other program {prec}")
    assert_bitexact_f32(d, c, f"other program {prec}")
    a, b = _both(rg, sess, x2, f"mlp {prec} 40 rows")
    assert_bitexact_f32(b, a, f"mlp {prec} 40 rows (second, smaller)")
    sess.close()
    sess2.close()


def test_noalloc_small_gemm_k_slices(rg, ref):
    """A Linear on the small-tile GEMM with K slices (4096 -> 256 at 16 and
    12 rows: eight slices meeting in 64-bit sum words in the slot set, which
    every allocation-free call zeroes in the shared scratch)."""
    from rustgears_amd import nn
    layers = _mlp(rg, [1024, 4096, 256], nn.Relu, seed=12)
    other = _mlp(rg, [96, 200, 64], nn.Gelu, seed=6)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    sess2 = rg.InferenceSession.from_layers(other, rg.ExecutionProvider.mi355x_int8())
    for rows in (16, 12):
        x = rg.randn([rows, 1024])
        a, b = _both(rg, sess, x, f"k slices {rows} rows")
        assert_bitexact_f32(b, a, f"k slices {rows} rows")
        assert_bitexact_f32(b, ref.RefProgram(layers).run(x, parallel=True), f"k slices {rows} rows vs oracle")
        c, d = _both(rg, sess2, rg.randn([700, 96]), "other program")
        assert_bitexact_f32(d, c, "other program")
    sess.close()
    sess2.close()


@pytest.mark.parametrize("prec", ["int8", "fp16"])
def test_noalloc_matches_run_device_cnn(rg, ref, prec):
    from rustgears_amd import nn
    m = _cnn(rg, seed=11, stride=2).add(nn.Linear(32 * 3 * 3, 24)).add(nn.Relu()).add(nn.Linear(24, 10))
    layers = m.export()
    sess = rg.InferenceSession.from_layers(layers, _providers(rg)[prec])
    x1, x2 = rg.randn([6, 3, 14, 14]), rg.randn([2, 3, 14, 14])
    for x, what in ((x1, "6 images"), (x2, "2 images (second, smaller)")):
        a, b = _both(rg, sess, x, f"cnn {prec} {what}")
        assert_bitexact_f32(b, a, f"cnn {prec} {what}")
        if prec == "int8":
            assert_bitexact_f32(b, ref.RefProgram(layers).run(x, parallel=True), f"cnn int8 {what} vs oracle")
    sess.close()


def test_noalloc_refuses_shapes_beyond_the_scratch(rg):
    """1024 -> 4096 -> 16 on 8192 rows keeps a 128 MiB f32 activation between
    the Linears: more than the 64 MiB scratch.  The shape query refuses it
    (nothing is enqueued), so does the run, and a smaller shape then runs."""
    from rustgears_amd import nn
    from rustgears_amd import _native as N
    from rustgears_amd.inference import DeviceBuffer
    rg.manual_seed(3)
    layers = nn.Sequential().add(nn.Linear(1024, 4096)).add(nn.Relu()).add(nn.Linear(4096, 16)).export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    st, _ = _noalloc(sess, None, (8192, 1024), None)
    assert st == ERR_CAPACITY, st
    assert "device scratch" in N.lib().rgnpu_last_error().decode()
    x = rg.randn([8192, 1024])
    d_x, d_y = DeviceBuffer.from_array(x), DeviceBuffer(8192 * 16 * 4)
    st, _ = _noalloc(sess, d_x, x.shape, d_y)
    assert st == ERR_CAPACITY, st
    a, b = _both(rg, sess, x[:500], "after the refusal, 500 rows")
    assert_bitexact_f32(b, a, "after the refusal")
    sess.close()


def test_noalloc_leaves_the_profile_and_refuses_capture(rg):
    from rustgears_amd import nn
    from rustgears_amd.inference import DeviceBuffer
    layers = _mlp(rg, [64, 128, 32], nn.Relu, seed=9)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    x = rg.randn([100, 64])
    sess.run(x)
    before = [r.macs for r in sess.last_npu_profile().records]
    x2 = rg.randn([30, 64])
    d_x, d_y = DeviceBuffer.from_array(x2), DeviceBuffer(30 * 32 * 4)
    assert _noalloc(sess, d_x, x2.shape, d_y)[0] == 0
    sess.synchronize()
    assert [r.macs for r in sess.last_npu_profile().records] == before
    sess.set_capture(True)
    assert _noalloc(sess, d_x, x2.shape, d_y)[0] == 1
    sess.close()
