"""Production taps: the kernels the benchmark times, checked operand by operand.

Capture mode switches kernels to their capture forms (exact GELU everywhere,
no conv + pool fusion, every f32 output stored).  Production taps
(set_capture("production"), RGNPU_CAPTURE_PRODUCTION) keep the production
plan and kernels unchanged and copy, device to device between launches, what
exists in memory after each op:

* the i8 operand a Linear's GEMM read -- written by the one-pass input
  quantization (npu.rs:312 -> quantize.rs:18-24 on the run's input) or by the
  previous GEMM's fused requantization, with the certified GELU form for
  GELU producers;
* the scale every quantizing op derived from its absmax slot (per tensor for
  a Linear, per image for a conv, npu.rs:346-351); a one-row GEMV that
  measures its own input's absmax keeps it in registers, so it has none;
* the f32 output of every op that stores one (a conv + pool kernel stores
  only the pooled output, the MaxPool2d op's; the CNN's two conv + pool
  stages run as one kernel that keeps the first pool's output in LDS).

Each is compared bit for bit with the oracle's capture of the same op, at
the benchmark's full sizes: the 4 x 4096^2 GELU stack (8192 rows), the deep
MLP (4096 rows), the CNN (256 images), the decode-shape GEMVs (one and
eight rows) and the quickstart MLP (64 rows).
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def _check_production(rg, ref, layers, x, what, want_q, want_out, no_scale=()):
    """Runs the production path with taps and the oracle with capture; checks
    every available tap and that exactly the expected ones exist (want_q /
    want_out: op indices with an i8 operand / an f32 output in memory;
    no_scale: quantizing ops whose absmax no slot holds)."""
    print(f"[taps] {what} x{tuple(x.shape)}", flush=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y_plain = sess.run(x)
    sess.set_capture("production")
    y = sess.run(x)
    prof = sess.last_npu_profile()
    prog = ref.RefProgram(layers)
    prog.set_capture(True)
    yr = prog.run(x, parallel=True)
    assert sess.op_labels() == prog.labels(), what
    have_q, have_out, checked = [], [], 0
    for i in range(prog.num_ops):
        tag = f"{what} op{i} ({prog.labels()[i]})"
        assert sess.capture(i, 2).size == 0, tag + ": no i32 sums on the production path"
        q = sess.capture(i, 0)
        if q.size:
            have_q.append(i)
            want = prog.capture(i, 0)
            assert q.shape == want.shape and np.array_equal(q, want), \
                f"{tag} qact: {np.count_nonzero(q != want)} of {want.size} differ"
            checked += q.size
        s = sess.capture(i, 1)
        ws = prog.capture(i, 1)
        if i in no_scale:
            assert ws.size and s.size == 0, tag + ": the scale is not in memory"
        elif ws.size:
            assert_bitexact_f32(s, ws, tag + " scale")
        o = sess.capture(i, 3)
        if o.size:
            have_out.append(i)
            assert_bitexact_f32(o, prog.capture(i, 3), tag + " out")
    assert have_q == want_q, (what, have_q)
    assert have_out == want_out, (what, have_out)
    assert_bitexact_f32(y, yr, what + " output")
    assert_bitexact_f32(y_plain, yr, what + " output without taps")
    sess.close()
    print(f"[taps] {what}: {checked} i8 operand bytes bit-exact", flush=True)
    return prof


def test_linear_stack_production_operands(rg, ref):
    """S: layer 1's operand from the one-pass input quantization, layers 2-4's
    from the fused requantization with the certified GELU; only the last
    layer stores an f32 output."""
    from rustgears_amd import configs
    model, x = configs.linear_stack()
    prof = _check_production(rg, ref, model.export(), x, "stack 4x4096 gelu", [0, 1, 2, 3], [3])
    for r in prof.records[1:]:
        assert r.duration_ns == r.kernel_ns, r  # fused: nothing launched before the GEMM


def test_deep_mlp_production_operands(rg, ref):
    """D: 784 -> 1024 quantizes its own input in one pass; the 1024 -> 1024
    layer and the head read operands from their producers' requantization."""
    from rustgears_amd import configs
    model, x = configs.deep_mlp()
    _check_production(rg, ref, model.export(), x, "deep mlp", [0, 1, 2], [2])


def test_cnn_production_operands(rg, ref):
    """C: both convs run as one kernel per image (conv_pool_pair_kernel):
    conv1 quantizes its f32 image into LDS, pools into LDS, and conv2
    quantizes those pooled planes and pools into memory, so neither conv's
    output nor pool 1's is in memory (pool 2's is); the per-image scales come
    from conv1's own absmax and from the pooled planes' absmax, both written
    to the convs' slots; the fc layer and the head quantize their inputs as
    they read them (with pool 2's and the fc layer's absmax), so no i8
    operand is in memory; their scales and outputs are."""
    from rustgears_amd import configs
    model, x = configs.cnn()
    layers = model.export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    labels = sess.op_labels()
    sess.close()
    # conv, pool, conv, pool, flatten, fc, head
    assert [l.split("(")[0] for l in labels] == ["NPU::FusedConv2dAct", "NPU::MaxPool2d", "NPU::FusedConv2dAct",
                                                 "NPU::MaxPool2d", "NPU::Flatten", "NPU::FusedGemmAct",
                                                 "NPU::Gemm"], labels
    _check_production(rg, ref, layers, x, "cnn", [], [3, 4, 5, 6])


@pytest.mark.parametrize("batch,want_q,no_scale", [(1, [1], [0]), (8, [0, 1], [])], ids=["b1", "b8"])
def test_gemv_production_operands(rg, ref, batch, want_q, no_scale):
    """G (8192 -> 28672 SiLU -> 8192): at one row, layer 1 measures and
    quantizes its own input as it stages it (neither its operand nor its
    absmax is in memory) and quant_rows writes layer 2's operand from layer
    1's output; at eight rows the one-pass input quantization writes layer
    1's operand and quant_rows layer 2's, both read by the matrix-core GEMV.
    Both layers' f32 outputs are in memory."""
    from rustgears_amd import configs
    layers, x = configs.gemv(batch=batch)
    _check_production(rg, ref, layers, x, f"gemv b{batch}", want_q, [0, 1], no_scale)


def test_quickstart_production_operands(rg, ref):
    """Q (64 rows, 4 -> 32 + BN + ReLU -> 3) runs as one workgroup: both
    operands and the hidden activations stay in LDS, only the program's
    output is in memory; each layer's absmax is written to its slot, so both
    scales are tapped."""
    from rustgears_amd import configs
    model, x = configs.quickstart()
    _check_production(rg, ref, model.export(), x, "quickstart", [], [1])


@pytest.mark.parametrize("rows,k", [(1024, 1024), (2048, 1536), (3072, 2048), (4096, 3072), (6144, 4096)],
                         ids=["U4", "U8", "U16", "U32", "U64"])
def test_input_quantization_every_grid_shape(rg, ref, rows, k):
    """The one-pass input quantization keeps U = 4, 8, 16, 32 or 64 units
    per thread, the smallest whose grid fits one workgroup per CU (192
    workgroups here, 128 for U = 4): a Linear(k, 40) + ReLU on rows x k
    inputs that select each U, its i8 operand, scale and output bit-exact
    with the oracle's."""
    from rustgears_amd import nn
    rg.manual_seed(rows + k)
    layers = nn.Sequential().add(nn.Linear(k, 40)).add(nn.Relu()).export()
    x = rg.randn([rows, k])
    x[rows // 3, k - 1] = -41.5  # the absmax in the last unit of one row
    _check_production(rg, ref, layers, x, f"input quant {rows}x{k}", [0], [0])
