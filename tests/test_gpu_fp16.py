"""NpuPrecision::Fp16 on the MI355X provider against the CPU oracle.

The reference (npu.rs:425-445) sums round_fp16(x) * w serially in f32 and
returns act(round_fp16(acc + bias)).  The products of two fp16 values are
exact in f32, so the MFMA path differs only in summation order, and parity
is a bound, not bit equality (unlike INT8):
  |acc_gpu - acc_ref| <= E = 2 K 2^-24 sum_k |p_k|
(any f32 summation order is within (K-1) u sum|p| of the exact sum, so two
orders are within twice that), round_fp16 then moves each value by at most
one fp16 ulp (2^-10 relative), and the activation scales the difference by
at most 1.13 (GELU's largest slope; 1 for ReLU/None).  Each op is checked on
its own: the oracle runs that op on the GPU's own captured input, so errors
do not compound.  The elementwise lone ChannelAffine must match bit for bit.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu

CAP_OUT = 3


def make_session(rg, layers):
    return rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_fp16())


def fp16_ulp(v):
    v = np.maximum(np.abs(v.astype(np.float64)), 2.0**-14)
    return np.exp2(np.floor(np.log2(v)) - 10)


def check_op_bound(ref, got, want, a, w_rounded, slope, what):
    """got/want [m, n]; a [m, k] op input; w_rounded [n, k]."""
    ah = ref.round_fp16(a).astype(np.float64)
    sum_abs = np.abs(ah) @ np.abs(w_rounded.astype(np.float64)).T
    k = a.shape[1]
    e = 2.0 * k * 2.0**-24 * sum_abs
    bound = slope * (fp16_ulp(want) + e) + 1e-30
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = np.flatnonzero(~(diff <= bound))
    assert bad.size == 0, (f"{what}: {bad.size} outside the bound, first {bad[:5]} got {got.ravel()[bad[:5]]} "
                           f"want {want.ravel()[bad[:5]]} bound {bound.ravel()[bad[:5]]}")
    exact = np.mean(got.view(np.uint32) == want.view(np.uint32))
    print(f"[fp16] {what}: max |diff| {diff.max():.3g}, bit-equal {exact:.4f}", flush=True)
    return exact


def linear_groups(layers):
    """Split a layer list into the reference's fused ops (Linear/Conv2d plus a
    following Activation; BatchNorm exports a ChannelAffine that folds into
    the layer before it)."""
    from rustgears_amd.inference import LayerSpec
    groups, i = [], 0
    while i < len(layers):
        g = [layers[i]]
        i += 1
        if isinstance(g[0], (LayerSpec.Linear, LayerSpec.Conv2d)):
            while i < len(layers) and isinstance(layers[i], LayerSpec.ChannelAffine):
                g.append(layers[i])
                i += 1
            if i < len(layers) and isinstance(layers[i], LayerSpec.Activation):
                g.append(layers[i])
                i += 1
        groups.append(g)
    return groups


def check_per_op(rg, ref, layers, x, what, slope=1.13, min_exact=0.5):
    from rustgears_amd.inference import LayerSpec
    print(f"[fp16] {what} x{tuple(x.shape)}", flush=True)
    sess = make_session(rg, layers)
    sess.set_capture(True)
    y = sess.run(x)
    groups = linear_groups(layers)
    p_all = ref.RefProgram(layers, precision=ref.FP16)
    assert sess.op_labels() == p_all.labels() and len(groups) == p_all.num_ops, what
    inp = x
    for i, g in enumerate(groups):
        p = ref.RefProgram(g, precision=ref.FP16)
        want = p.run(inp)
        got = sess.capture(i, CAP_OUT)
        assert got.size == want.size, f"{what} op{i}"
        got = got.reshape(want.shape)
        head = g[0]
        if isinstance(head, LayerSpec.Linear):
            a = inp.reshape(-1, head.in_features)
            w = ref.round_fp16(p.op_weight_fp16(0))
            check_op_bound(ref, got.reshape(a.shape[0], -1), want.reshape(a.shape[0], -1), a, w, slope,
                           f"{what} op{i}")
        elif isinstance(head, LayerSpec.Conv2d):
            n, c = inp.shape[0], inp.shape[1]
            k, s, pd, o = head.kernel, head.stride, head.padding, head.out_channels
            oh, ow = got.shape[2], got.shape[3]
            xp = np.pad(inp, ((0, 0), (0, 0), (pd, pd), (pd, pd)))
            cols = np.empty((n, oh * ow, c * k * k), np.float32)
            for ci in range(c):
                for ki in range(k):
                    for kj in range(k):
                        patch = xp[:, ci, ki:ki + s * oh:s, kj:kj + s * ow:s]
                        cols[:, :, (ci * k + ki) * k + kj] = patch.reshape(n, -1)
            w = ref.round_fp16(p.op_weight_fp16(0))
            g2 = got.transpose(0, 2, 3, 1).reshape(-1, o)
            w2 = want.transpose(0, 2, 3, 1).reshape(-1, o)
            check_op_bound(ref, np.ascontiguousarray(g2), np.ascontiguousarray(w2), cols.reshape(-1, c * k * k), w,
                           slope, f"{what} op{i}")
        else:
            assert_bitexact_f32(got, want, f"{what} op{i}")
        inp = got
    prof = sess.last_npu_profile()
    assert str(prof.precision) == "FP16"
    assert prof.fp32_weight_bytes == p_all.fp32_bytes and prof.npu_weight_bytes == p_all.npu_bytes
    sess.close()
    return y


def test_fp16_mlp_per_op(rg, ref):
    from rustgears_amd import configs
    model, x = configs.deep_mlp(rows=300)
    check_per_op(rg, ref, model.export(), x, "deep_mlp fp16")


@pytest.mark.parametrize("act", ["relu", "gelu", "none", "sigmoid"])
def test_fp16_linear_activations(rg, ref, act):
    from rustgears_amd import nn
    rg.manual_seed(3)
    m = nn.Sequential().add(nn.Linear(200, 300))
    if act != "none":
        m.add({"relu": nn.Relu, "gelu": nn.Gelu, "sigmoid": nn.Sigmoid}[act]())
    m.add(nn.Linear(300, 7))
    check_per_op(rg, ref, m.export(), (rg.randn([37, 200]) * 3).astype(np.float32), f"linear {act}")


@pytest.mark.parametrize("rows", [1, 8, 255, 257, 1000, 4100])
def test_fp16_rows_and_split_k(rg, ref, rows):
    """Row counts around the 256-row tile and small batches (FP16 always uses
    the MFMA GEMM; few tiles take the split-K path)."""
    from rustgears_amd import nn
    rg.manual_seed(rows)
    m = nn.Sequential().add(nn.Linear(1000, 500)).add(nn.Relu()).add(nn.Linear(500, 33))
    check_per_op(rg, ref, m.export(), rg.randn([rows, 1000]), f"rows {rows}")


def test_fp16_cnn_per_op(rg, ref):
    from rustgears_amd import configs
    model, x = configs.cnn(n=16)
    check_per_op(rg, ref, model.export(), x, "cnn fp16")


def test_fp16_conv_stride_padding(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(11)
    m = (nn.Sequential().add(nn.Conv2d(5, 7, 3).stride(2).padding(1)).add(nn.Gelu())
         .add(nn.Conv2d(7, 4, 2)).add(nn.Flatten()).add(nn.Linear(4 * 4 * 4, 6)))
    check_per_op(rg, ref, m.export(), rg.randn([3, 5, 9, 9]), "conv s2 p1")


def test_fp16_lone_channel_affine_and_standalone_ops(rg, ref):
    from rustgears_amd.inference import Activation, LayerSpec
    rg.manual_seed(12)
    layers = [LayerSpec.ChannelAffine(rg.randn([10]), rg.randn([10])), LayerSpec.Activation(Activation.GELU),
              LayerSpec.Linear(10, 6, rg.randn([60]), rg.randn([6])), LayerSpec.Softmax()]
    x = (rg.randn([9, 10]) * 5).astype(np.float32)
    sess = make_session(rg, layers)
    sess.set_capture(True)
    sess.run(x)
    p = ref.RefProgram(layers[:1], precision=ref.FP16)
    want = p.run(x)
    assert_bitexact_f32(sess.capture(0, CAP_OUT).reshape(want.shape), want, "affine fp16")
    sess.close()
    check_per_op(rg, ref, layers, x, "affine/act/linear/softmax")


def test_fp16_special_values(rg, ref):
    """Inputs past the fp16 range and NaN: round_fp16 clamps them to
    +-65504 (npu.rs:442 path), so the outputs stay finite like the
    reference's."""
    from rustgears_amd import nn
    rg.manual_seed(8)
    m = nn.Sequential().add(nn.Linear(16, 8)).add(nn.Relu()).add(nn.Linear(8, 4))
    x = rg.randn([6, 16])
    x[0, 3] = np.nan
    x[1, 2] = np.inf
    x[2, :] = 1e6
    x[3, :] = 0.0
    x[4, 5] = 1e-9
    check_per_op(rg, ref, m.export(), x, "special values")


def test_fp16_report_and_accounting(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(0)
    model = nn.Sequential().add(nn.Linear(16, 64)).add(nn.BatchNorm1d(64)).add(nn.Relu()).add(nn.Linear(64, 4))
    layers = model.export()
    sess = make_session(rg, layers)
    p = ref.RefProgram(layers, precision=ref.FP16)
    rep = sess.compilation_report()
    assert "(FP16)" in rep and f"{p.fp32_bytes} B -> {p.npu_bytes} B" in rep, rep
    assert p.npu_bytes == (16 * 64 + 64 + 64 * 4 + 4) * 2
    sess.close()


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_fp16_gemv_decode_shape(rg, ref, batch):
    """The decode-shape config (SiLU then a plain Linear) scaled down, through
    the binary16 GEMV (batch <= 8)."""
    from rustgears_amd import configs
    layers, x = configs.gemv(batch=batch, d=1024, h=3584)
    check_per_op(rg, ref, layers, x, f"gemv fp16 b{batch}")


@pytest.mark.parametrize("spec", [(3, 32, 3, 1, 1), (2, 5, 3, 2, 0), (1, 64, 5, 1, 2), (7, 4, 2, 1, 0), (3, 17, 3, 3, 1)])
def test_fp16_direct_conv_exact(rg, ref, spec):
    """A convolution whose window holds at most 32 values runs as a direct
    conv that sums the taps in the reference's serial im2col order, so it is
    bit-exact with the oracle (not only within the reordering bound)."""
    from rustgears_amd import nn
    C, O, k, s, p = spec
    rg.manual_seed(C * 100 + O * 10 + k)
    m = nn.Sequential().add(nn.Conv2d(C, O, k).stride(s).padding(p)).add(nn.Relu())
    layers = m.export()
    x = (rg.randn([4, C, 11, 13]) * 2.0).astype(np.float32)
    print(f"[direct conv fp16] {spec}", flush=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_fp16())
    y = sess.run(x)
    want = ref.RefProgram(layers, precision=ref.FP16).run(x)
    assert_bitexact_f32(y, want, f"direct conv {spec}")
    sess.close()


@pytest.mark.parametrize("seed", range(32))
def test_fp16_random_models(rg, ref, seed):
    """The INT8 suite's seeded random layer stacks on this provider: every
    Linear/Conv op within the summation-order bound, every other op bit for
    bit."""
    from test_gpu_parity import _random_model
    layers, x = _random_model(1000 + seed)
    check_per_op(rg, ref, layers, x, f"random model {seed}")


HANDOFF_CASES = [
    # (name, dims, act, rows): the tile shape of the producer GEMMs in the comment
    ("stack 256x256 gelu", [4096, 4096, 4096, 4096], "gelu", 8192),  # S's shape, 3 hand-offs
    ("256x128 relu ragged", [1000, 3000, 2004, 20], "relu", 2600),    # then 128x128; N = 2004 pads to 2048
    ("128x128 tanh", [700, 1024, 516, 300], "tanh", 2048),            # 1024 -> 516 splits K: converts
]


@pytest.mark.parametrize("name,dims,act,rows", HANDOFF_CASES, ids=[c[0] for c in HANDOFF_CASES])
def test_fp16_operand_handoff_is_bit_identical(rg, monkeypatch, name, dims, act, rows):
    """An FP16 Linear whose next op is an FP16 Linear on the same rows writes
    that Linear's binary16 operand from its GEMM epilogue (the consumer's
    conversion pass is gone): outputs bit-identical to RGNPU_F16_HANDOFF=0,
    and a consumer fed this way launches nothing before its GEMM.  With GELU
    the hand-off certifies the operand from gelu_approx: every mode of
    RGNPU_GELU_CERT (1 certified, 3 a margin that queues ~1% of the values
    for the exact GELU, 2 every value uncertain so each wave redoes its walk
    exactly, 0 exact) must give the same bits."""
    from rustgears_amd import nn
    rg.manual_seed(rows + len(dims))
    act_cls = {"gelu": nn.Gelu, "relu": nn.Relu, "tanh": nn.Tanh}[act]
    m = nn.Sequential()
    for a, b in zip(dims[:-1], dims[1:]):
        m.add(nn.Linear(a, b)).add(act_cls())
    layers = m.export()
    x = rg.randn([rows, dims[0]])
    runs = [("0", "1"), ("1", "1")] + ([("1", "3"), ("1", "2"), ("1", "0")] if act == "gelu" else [])
    outs, profs = {}, {}
    for handoff, cert in runs:
        monkeypatch.setenv("RGNPU_F16_HANDOFF", handoff)
        monkeypatch.setenv("RGNPU_GELU_CERT", cert)
        print(f"[fp16-handoff] {name} handoff {handoff} cert {cert}", flush=True)
        sess = make_session(rg, layers)
        y = sess.run(x)
        y2 = sess.run(x)
        profs[handoff, cert] = sess.last_npu_profile()
        sess.close()
        assert_bitexact_f32(y2, y, f"{name} handoff {handoff} cert {cert} second run")
        outs[handoff, cert] = y
    for key in runs[1:]:
        assert_bitexact_f32(outs[key], outs["0", "1"], f"{name}: hand-off (cert {key[1]}) vs conversion pass")
    gemms = [r for r in profs["1", "1"].records if "Gemm" in r.op]
    assert gemms[1].duration_ns == gemms[1].kernel_ns, gemms  # no conversion before the second GEMM
    gemms0 = [r for r in profs["0", "1"].records if "Gemm" in r.op]
    assert gemms0[1].duration_ns > gemms0[1].kernel_ns, gemms0
