"""INT8 Linears with few output tiles, quantizing their input as they read it
(kernels.hip gemm_xq_small_kernel, program.cpp make_plan small_xq).

A Linear whose GEMM would otherwise have fewer than 128 tiles of 128 x 128
and whose input's absmax its producer emitted (npu.rs:312 ->
quantize.rs:18-24 with that absmax) runs as one kernel: one workgroup per
16 x 16 (or 16 x 64) output block and K slice, quantizing the f32 input as
it loads it, adding its waves' exact i32 sums in LDS, the K slices meeting
in one 64-bit counting atomic per output (the thread that completes the
count applies the fused epilogue, quantize.rs:104-113).  Each case's output must equal bit for bit the
oracle's and the output with the kernel turned off (RGNPU_SMALL_XQ=0:
quant_rows, the tile GEMM and, when it splits K, its epilogue): the CNN's fc
layer, one, four and eight K slices, both block widths, slices staged in
LDS in one and in two chunks (the second partial, K ending inside it) and
slices short enough for register loads, ragged rows (the last 16-row block
partly filled), K not a multiple of 64, N not a multiple of 16,
every activation, and inputs that drive the scale to infinity or the
activations to NaN.  Programs it does not take (K % 4 != 0, 128 tiles or
more) run the tile GEMM.  The op's record has no launch before its GEMM when
the kernel runs.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def _chain(rg, dims, acts, seed):
    from rustgears_amd import nn
    from rustgears_amd.inference import Activation, LayerSpec
    rg.manual_seed(seed)
    layers = []
    mods = {"relu": nn.Relu, "sigmoid": nn.Sigmoid, "tanh": nn.Tanh, "gelu": nn.Gelu}
    for i in range(len(dims) - 1):
        layers += nn.Linear(dims[i], dims[i + 1]).export()
        a = acts[i]
        if a == "silu":
            layers.append(LayerSpec.Activation(Activation.SILU))
        elif a == "leaky":
            layers += nn.LeakyRelu(0.05).export()
        elif a is not None:
            layers += mods[a]().export()
    return layers


def _run(rg, layers, x, on, monkeypatch):
    if on:
        monkeypatch.delenv("RGNPU_SMALL_XQ", raising=False)
    else:
        monkeypatch.setenv("RGNPU_SMALL_XQ", "0")
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    y2 = sess.run(x)
    recs = list(sess.last_npu_profile().records)
    sess.close()
    monkeypatch.delenv("RGNPU_SMALL_XQ", raising=False)
    assert_bitexact_f32(y2, y, "second run")
    return y, recs


def _check(rg, ref, monkeypatch, layers, x, what, taken):
    """taken: op indices expected to run gemm_xq_small_kernel."""
    print(f"[small-xq] {what} x{tuple(x.shape)}", flush=True)
    want = ref.RefProgram(layers).run(x, parallel=True)
    y, recs = _run(rg, layers, x, True, monkeypatch)
    y0, recs0 = _run(rg, layers, x, False, monkeypatch)
    assert_bitexact_f32(y, want, f"{what} (small GEMM) vs oracle")
    assert_bitexact_f32(y0, want, f"{what} (tile GEMM) vs oracle")
    assert [r.op for r in recs] == [r.op for r in recs0]
    for i in taken:
        r, r0 = recs[i], recs0[i]
        assert r.kernel_ns > 0 and r.duration_ns == r.kernel_ns, (what, i, r)
        assert r0.duration_ns > r0.kernel_ns, (what, i, r0)  # quant_rows before the tile GEMM
        print(f"[small-xq]   op{i}: {r.kernel_ns / 1e3:.1f} us, off {r0.duration_ns / 1e3:.1f} us", flush=True)
    return recs


def test_cnn_fc_layer(rg, ref, monkeypatch):
    from rustgears_amd import configs
    model, x = configs.cnn()
    layers = model.export()
    recs = _check(rg, ref, monkeypatch, layers, x, "cnn[256,3,32,32]", taken=[5])
    assert recs[5].op.startswith("NPU::FusedGemmAct"), [r.op for r in recs]


CASES = [
    # (rows, dims, acts, ops taking the kernel).  Each first Linear splits K,
    # and a Linear whose GEMM is not split hands the next Linear its i8
    # operand only when its N is a multiple of 4 (fused requantization).
    # The kernel's geometry (block width, K slices) is noted per op.
    (64, (512, 2048, 1024, 384), ("relu", "gelu", None), [1, 2]),  # 64 x 4 slices; 16 x 1
    (200, (512, 300, 102), ("tanh", "silu"), [1]),                  # 16 x 1: ragged rows, K 300, N 102
    (17, (1024, 4096, 2048, 16), ("leaky", "sigmoid", "relu"), [1]),  # 64 x 4
    (16, (1024, 4096, 256), ("relu", "relu"), [1]),                 # 16 x 8
    (1000, (1024, 256, 160), ("relu", "leaky"), [1]),               # 64 x 1 (252 blocks)
    (256, (1024, 7932, 256), ("relu", None), [1]),                   # 64 x 4: two LDS chunks, K 7932
]


@pytest.mark.parametrize("rows,dims,acts,taken", CASES,
                         ids=[f"m{r}-" + "x".join(map(str, d)) for r, d, _, _ in CASES])
def test_chains(rg, ref, monkeypatch, rows, dims, acts, taken):
    layers = _chain(rg, dims, acts, seed=rows + len(dims))
    x = rg.randn([rows, dims[0]]) * np.float32(1.5)
    _check(rg, ref, monkeypatch, layers, x, f"chain m={rows} {dims}", taken)


def test_special_values(rg, ref, monkeypatch):
    """Eight K slices.  An infinite input makes the first Linear's scale
    infinite and its outputs NaN (0 * inf), which the second Linear's absmax
    ignores; a huge finite input overflows the first Linear's outputs to
    infinity, so the second Linear's scale is infinite and its sums'
    products NaN; an all-zero input gives scale 1 throughout."""
    layers = _chain(rg, (512, 2048, 384), (None, "relu"), seed=3)
    for what, fill in (("inf", np.inf), ("huge", 3e38), ("zeros", 0.0)):
        x = rg.randn([48, 512])
        if what == "zeros":
            x[:] = 0.0
        else:
            x[5, 7] = fill
            x[11, 200] = -fill
        _check(rg, ref, monkeypatch, layers, x, f"special {what}", [1])


NOT_TAKEN = [
    # (what, rows, dims): the tile GEMM runs
    ("K % 4 != 0", 40, (512, 130, 200)),
    ("128 tiles", 4096, (1024, 256, 512)),
]


@pytest.mark.parametrize("what,rows,dims", NOT_TAKEN, ids=[w for w, _, _ in NOT_TAKEN])
def test_programs_it_does_not_take(rg, ref, monkeypatch, what, rows, dims):
    layers = _chain(rg, dims, ("relu", None), seed=21)
    print(f"[small-xq] not taken: {what}", flush=True)
    x = rg.randn([rows, dims[0]])
    want = ref.RefProgram(layers).run(x, parallel=True)
    y, _ = _run(rg, layers, x, True, monkeypatch)
    assert_bitexact_f32(y, want, what)
