"""GPU parity: the MI355X provider against the CPU oracle, bit for bit.

Every test runs the HIP path through the C ABI (librgnpu.so) and compares,
per fused op, the captured i8 activations, activation scale(s), i32
accumulators and f32 outputs with the oracle's restatement of
NpuProgram::execute (npu.rs:296-421).  The bar is bit-exact for all four,
including f32 (the fused epilogue and activations reproduce the reference's
f32 arithmetic and libm exactly), which is stricter than the 1e-5 relative
tolerance the target allows; argmax equality follows.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def make_session(rg, layers):
    return rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())


def check_against_oracle(rg, ref, layers, x, what="", parallel=True):
    print(f"[parity] {what} x{tuple(x.shape)}", flush=True)
    sess = make_session(rg, layers)
    sess.set_capture(True)
    y = sess.run(x)
    p = ref.RefProgram(layers)
    p.set_capture(True)
    yr = p.run(x, parallel=parallel)
    assert sess.op_labels() == p.labels(), what
    assert y.shape == yr.shape, what
    for i in range(p.num_ops):
        for cap, name in ((0, "qact"), (1, "scale"), (2, "acc"), (3, "out")):
            want = p.capture(i, cap)
            if want.size == 0 and cap != 3:
                continue
            got = sess.capture(i, cap)
            tag = f"{what} op{i} ({p.labels()[i]}) {name}"
            if want.dtype == np.float32:
                assert_bitexact_f32(got, want, tag)
            else:
                assert got.shape == want.shape, tag
                if not np.array_equal(got, want):
                    bad = np.flatnonzero(got != want)
                    raise AssertionError(f"{tag}: {bad.size} differ, first {bad[:5]} got {got[bad[:5]]} "
                                         f"want {want[bad[:5]]}")
    assert_bitexact_f32(y, yr, what + " output")
    if y.ndim == 2 and y.shape[1] > 1 and y.shape[0] > 0:
        assert np.array_equal(np.argmax(y, 1), np.argmax(yr, 1))
    prof = sess.last_npu_profile()
    assert prof is not None and prof.fused_ops == p.num_ops and prof.original_layers == p.original_layers
    assert [r.op for r in prof.records] == p.labels()
    assert [r.macs for r in prof.records] == [p.op_macs(i) for i in range(p.num_ops)]
    assert prof.fp32_weight_bytes == p.fp32_bytes and prof.npu_weight_bytes == p.npu_bytes
    sess.close()
    return y


def test_golden_fixtures(rg, ref):
    import golden_cases
    for case in golden_cases.load_all():
        print(f"[golden] {case['name']}", flush=True)
        sess = make_session(rg, case["layers"])
        sess.set_capture(True)
        y = sess.run(case["x"])
        assert sess.op_labels() == case["labels"]
        assert_bitexact_f32(y, case["y"], case["name"])
        for i, caps in enumerate(case["caps"]):
            for what, arr in caps.items():
                got = sess.capture(i, what)
                if arr.dtype == np.float32:
                    assert_bitexact_f32(got, arr, f"{case['name']} op{i} cap{what}")
                else:
                    assert np.array_equal(got, arr), f"{case['name']} op{i} cap{what}"
        sess.close()


def test_quickstart_mlp(rg, ref):
    from rustgears_amd import configs
    model, x = configs.quickstart()
    check_against_oracle(rg, ref, model.export(), x, "quickstart")


def test_deep_mlp_full(rg, ref):
    from rustgears_amd import configs
    model, x = configs.deep_mlp()
    check_against_oracle(rg, ref, model.export(), x, "deep_mlp[4096,784]")


def test_cnn_full(rg, ref):
    from rustgears_amd import configs
    model, x = configs.cnn()
    check_against_oracle(rg, ref, model.export(), x, "cnn[256,3,32,32]")


def test_linear_stack_gelu_scaled(rg, ref):
    from rustgears_amd import configs
    model, x = configs.linear_stack(rows=384, width=640, depth=4)
    check_against_oracle(rg, ref, model.export(), x, "stack 640 gelu")


def test_linear_stack_gelu_full(rg, ref):
    """The 4096^2 x 4 GELU stack at its benchmark size (8192 rows), through
    the large-tile GEMM, bit-exact against the oracle."""
    from rustgears_amd import configs
    model, x = configs.linear_stack()
    check_against_oracle(rg, ref, model.export(), x, "stack 4096 gelu full")


def test_large_tile_gemm_ragged(rg, ref):
    """Ragged M, N and K on the large-tile kernel (>= 256 tiles of 256x128)."""
    from rustgears_amd import nn
    rg.manual_seed(41)
    model = nn.Sequential().add(nn.Linear(1000, 4000)).add(nn.Relu()).add(nn.Linear(4000, 37))
    check_against_oracle(rg, ref, model.export(), rg.randn([4100, 1000]), "big ragged")


@pytest.mark.parametrize("batch", [1, 8])
def test_gemv_silu_full(rg, ref, batch):
    """The decode-shape GEMV config at full size (8192 -> 28672 SiLU -> 8192)."""
    from rustgears_amd import configs
    layers, x = configs.gemv(batch=batch)
    check_against_oracle(rg, ref, layers, x, f"gemv full b{batch}")


@pytest.mark.parametrize("batch", [1, 3, 8])
def test_gemv_relu_full(rg, ref, batch):
    """The ReLU twin of the decode-shape config, a model the reference itself
    can express (SiLU is the build's extension)."""
    from rustgears_amd import configs
    from rustgears_amd.inference import Activation
    layers, x = configs.gemv(batch=batch, act=Activation.RELU)
    check_against_oracle(rg, ref, layers, x, f"gemv relu full b{batch}")


@pytest.mark.parametrize("batch", [1, 8])
def test_gemv_silu_scaled(rg, ref, batch):
    from rustgears_amd import configs
    layers, x = configs.gemv(batch=batch, d=1024, h=3584)
    check_against_oracle(rg, ref, layers, x, f"gemv b{batch}")


@pytest.mark.parametrize("rows", [1, 2, 7, 8, 9, 16, 255, 256, 257])
def test_rows_around_gemv_and_tile_boundaries(rg, ref, rows):
    rg.manual_seed(rows)
    from rustgears_amd import nn
    model = nn.Sequential().add(nn.Linear(200, 130)).add(nn.Relu()).add(nn.Linear(130, 7))
    check_against_oracle(rg, ref, model.export(), rg.randn([rows, 200]), f"rows={rows}")


@pytest.mark.parametrize("k,n", [(1, 1), (3, 300), (64, 64), (127, 129), (1000, 5), (4100, 17)])
def test_ragged_k_and_n(rg, ref, k, n):
    rg.manual_seed(k * 7 + n)
    from rustgears_amd import nn
    model = nn.Sequential().add(nn.Linear(k, n)).add(nn.LeakyRelu(0.05))
    check_against_oracle(rg, ref, model.export(), rg.randn([33, k]), f"k={k} n={n}")


@pytest.mark.parametrize("k,n,rows,act", [(4, 1, 9, "none"), (100, 2, 300, "sigmoid"), (1024, 10, 4097, "none"),
                                          (1500, 7, 33, "gelu"), (3000, 16, 600, "relu"), (32, 3, 64, "tanh"),
                                          (2049, 16, 9, "silu"), (256, 12, 1000, "leaky")])
def test_narrow_outputs(rg, ref, k, n, rows, act):
    """Linear layers with at most 16 outputs (classifier heads) on more than
    8 rows, with their output absmax feeding a following Linear: ragged K
    below, at and above one 1 KiB chunk, every fused activation."""
    from rustgears_amd.inference import Activation, LayerSpec
    a = {"relu": Activation.RELU, "sigmoid": Activation.SIGMOID, "tanh": Activation.TANH, "gelu": Activation.GELU,
         "leaky": Activation.leaky_relu(0.1), "silu": Activation.SILU, "none": None}[act]
    rg.manual_seed(k + 31 * n + rows)
    layers = [LayerSpec.Linear(k, n, rg.randn([k * n]), rg.randn([n]))]
    if a is not None:
        layers.append(LayerSpec.Activation(a))
    layers.append(LayerSpec.Linear(n, 40, rg.randn([n * 40]), rg.randn([40])))
    check_against_oracle(rg, ref, layers, (rg.randn([rows, k]) * 2.0).astype(np.float32),
                         f"narrow k={k} n={n} rows={rows} {act}")


@pytest.mark.parametrize("act", ["relu", "sigmoid", "tanh", "gelu", "leaky", "silu", "none"])
def test_fused_activations(rg, ref, act):
    from rustgears_amd.inference import Activation, LayerSpec
    a = {"relu": Activation.RELU, "sigmoid": Activation.SIGMOID, "tanh": Activation.TANH, "gelu": Activation.GELU,
         "leaky": Activation.leaky_relu(0.01), "silu": Activation.SILU, "none": Activation.NONE}[act]
    rg.manual_seed(99)
    w, b = rg.randn([96 * 80]), rg.randn([80])
    layers = [LayerSpec.Linear(96, 80, w, b), LayerSpec.Activation(a), LayerSpec.Linear(80, 24, rg.randn([80 * 24]),
                                                                                     rg.randn([24]))]
    check_against_oracle(rg, ref, layers, (rg.randn([40, 96]) * 3).astype(np.float32), f"act {act}")


@pytest.mark.parametrize("spec", [(3, 8, 3, 1, 1), (4, 6, 3, 2, 0), (2, 5, 1, 1, 0), (3, 4, 2, 3, 1),
                                  (5, 7, 5, 2, 2)])
def test_conv_variants(rg, ref, spec):
    c, o, k, s, p = spec
    from rustgears_amd import nn
    rg.manual_seed(sum(spec))
    conv = nn.Conv2d(c, o, k).stride(s).padding(p)
    conv2 = nn.Conv2d(o, 6, 3).padding(1)
    model = nn.Sequential().add(conv).add(nn.Relu()).add(conv2).add(nn.Tanh())
    check_against_oracle(rg, ref, model.export(), rg.randn([5, c, 13, 11]), f"conv {spec}")


def test_pool_and_flatten_chain(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(5)
    model = (nn.Sequential().add(nn.Conv2d(2, 8, 3)).add(nn.Relu()).add(nn.MaxPool2d(3, 2)).add(nn.Conv2d(8, 4, 2))
             .add(nn.MaxPool2d(2)).add(nn.Flatten()).add(nn.Linear(4 * 2 * 2, 5)))
    check_against_oracle(rg, ref, model.export(), rg.randn([4, 2, 13, 13]), "pool chain")


def test_special_values(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(8)
    model = nn.Sequential().add(nn.Linear(16, 8)).add(nn.Relu()).add(nn.Linear(8, 4))
    layers = model.export()
    x = rg.randn([6, 16])
    x[0, 3] = np.nan
    x[1, :] = 0.0
    check_against_oracle(rg, ref, layers, x, "nan row")
    check_against_oracle(rg, ref, layers, np.zeros((3, 16), np.float32), "all zeros")
    check_against_oracle(rg, ref, layers, np.full((2, 16), 1e-13, np.float32), "tiny (scale 1)")


def test_standalone_ops(rg, ref):
    from rustgears_amd.inference import Activation, LayerSpec
    rg.manual_seed(12)
    layers = [LayerSpec.ChannelAffine(rg.randn([10]), rg.randn([10])), LayerSpec.Activation(Activation.GELU),
              LayerSpec.Linear(10, 6, rg.randn([60]), rg.randn([6])), LayerSpec.Softmax()]
    check_against_oracle(rg, ref, layers, rg.randn([9, 10]), "affine/act/softmax")
    check_against_oracle(rg, ref, [LayerSpec.Flatten()], rg.randn([2, 3, 4]), "flatten only")


def test_activation_math_sweep_on_device(rg, ref):
    """Standalone activation kernels over 2^22 f32 bit patterns spread over
    all binades (every 1024th pattern, plus an offset) against host libm."""
    from rustgears_amd.inference import Activation, LayerSpec
    bits = (np.arange(1 << 22, dtype=np.uint64) * 1024 + 517).astype(np.uint32)
    x = bits.view(np.float32).reshape(1 << 11, 1 << 11)
    for a in (Activation.TANH, Activation.SIGMOID, Activation.GELU, Activation.SILU):
        print(f"[sweep] {a}", flush=True)
        sess = make_session(rg, [LayerSpec.Activation(a)])
        y = sess.run(x)
        assert_bitexact_f32(y, ref.act_apply(a.code, 0.0, x), f"sweep {a}")
        sess.close()


def test_shape_changes_and_errors(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(3)
    layers = nn.Sequential().add(nn.Linear(12, 9)).add(nn.Relu()).export()
    sess = make_session(rg, layers)
    p = ref.RefProgram(layers)
    for rows in (5, 300, 1, 5):
        x = rg.randn([rows, 12])
        assert_bitexact_f32(sess.run(x), p.run(x), f"rows {rows}")
    with pytest.raises(rg.RgnpuError) as e:
        sess.run(np.ones((2, 13), np.float32))
    assert e.value.code == 2
    conv = make_session(rg, nn.Sequential().add(nn.Conv2d(3, 4, 3)).export())
    with pytest.raises(rg.RgnpuError):
        conv.run(np.ones((1, 2, 5, 5), np.float32))
    with pytest.raises(rg.RgnpuError):
        conv.run(np.ones((1, 3, 2, 2), np.float32))
    # the documented output-feature limit of a Linear layer (2^26)
    from rustgears_amd.inference import LayerSpec
    n_big = (1 << 26) + 1
    with pytest.raises(rg.RgnpuError) as e:
        make_session(rg, [LayerSpec.Linear(1, n_big, np.zeros(n_big, np.float32), np.zeros(n_big, np.float32))])
    assert "2^26" in str(e.value)


@pytest.mark.parametrize("prec", ["int8", "fp16", "fp32"])
def test_empty_batch(rg, ref, prec):
    """Zero rows or images: the reference's quantize of an empty tensor takes
    scale 1 (quantize.rs:19-21) and every op yields an empty output of the
    right shape.  Nothing is launched for the empty ops, capture taps are
    empty, and the session (and its absmax slots) stays exact for the
    non-empty runs that follow."""
    from rustgears_amd import nn
    from rustgears_amd.inference import Activation, LayerSpec
    provider = {"int8": rg.ExecutionProvider.mi355x_int8(), "fp16": rg.ExecutionProvider.mi355x_fp16(),
                "fp32": rg.ExecutionProvider.Gpu(0)}[prec]
    rg.manual_seed(41)
    mlp = nn.Sequential().add(nn.Linear(300, 260)).add(nn.Gelu()).add(nn.Linear(260, 7)).export()
    cnn = (nn.Sequential().add(nn.Conv2d(3, 8, 3).padding(1)).add(nn.Relu()).add(nn.MaxPool2d(2))
           .add(nn.Conv2d(8, 40, 3)).add(nn.MaxPool2d(2)).add(nn.Flatten()).add(nn.Linear(40, 5)).export())
    tail = mlp + [LayerSpec.Activation(Activation.TANH), LayerSpec.Softmax()]
    for name, layers, shape in (("mlp", mlp, (300,)), ("cnn", cnn, (3, 8, 8)), ("softmax tail", tail, (300,))):
        print(f"[parity] empty batch {prec} {name}", flush=True)
        sess = rg.InferenceSession.from_layers(layers, provider)
        p = ref.RefProgram(layers, precision={"int8": ref.INT8, "fp16": ref.FP16, "fp32": ref.FP32}[prec])
        x0 = np.zeros((0,) + shape, np.float32)
        x = rg.randn([5] + list(shape))
        want = sess.run(x)
        for capture in (False, True):
            sess.set_capture(capture)
            y0 = sess.run(x0)
            assert y0.shape == p.run(x0).shape and y0.size == 0, f"{name}: {y0.shape}"
            assert_bitexact_f32(sess.run(x), want, f"{name}: run after an empty one (capture {capture})")
        sess.set_capture(False)
        dx, dy = rg.DeviceBuffer(4), rg.DeviceBuffer(4)
        assert sess.run_device(dx, x0.shape, dy) == y0.shape
        sess.synchronize()
        if prec == "int8":
            assert_bitexact_f32(want, p.run(x), f"{name} vs oracle")
        sess.close()


class _OffsetView:
    """A device pointer 4 bytes into a DeviceBuffer (not 16-byte aligned)."""

    def __init__(self, buf, offset):
        self.ptr = buf.ptr + offset
        self.nbytes = buf.nbytes - offset


@pytest.mark.parametrize("prec", ["int8", "fp16", "fp32"])
def test_unaligned_device_input(rg, ref, prec):
    """Device inputs that are not 16-byte aligned take the scalar paths of
    the absmax, quantize, FP16 conversion and FP32 padding kernels; the
    results equal the aligned run bit for bit (and the oracle for INT8)."""
    from rustgears_amd import _native as N
    from rustgears_amd import nn
    provider = {"int8": rg.ExecutionProvider.mi355x_int8(), "fp16": rg.ExecutionProvider.mi355x_fp16(),
                "fp32": rg.ExecutionProvider.Gpu(0)}[prec]
    rg.manual_seed(57)
    layers = (nn.Sequential().add(nn.Linear(256, 300)).add(nn.Gelu()).add(nn.Linear(300, 12)).export())
    sess = rg.InferenceSession.from_layers(layers, provider)
    for rows in (1, 8, 300):
        print(f"[parity] unaligned input {prec} rows {rows}", flush=True)
        x = rg.randn([rows, 256])
        want = sess.run(x)
        raw = rg.DeviceBuffer(x.nbytes + 16)
        dx = _OffsetView(raw, 4)
        N.check(N.lib().rgnpu_memcpy_h2d(dx.ptr, x.ctypes.data, x.nbytes))
        dy = rg.DeviceBuffer(want.nbytes)
        sess.run_device(dx, x.shape, dy)
        sess.synchronize()
        assert_bitexact_f32(dy.download(want.shape), want, f"{prec} rows {rows}")
        if prec == "int8":
            assert_bitexact_f32(want, ref.RefProgram(layers).run(x), f"oracle rows {rows}")
    sess.close()


def test_device_resident_run_matches_host_run(rg, ref):
    from rustgears_amd import configs
    model, x = configs.deep_mlp(rows=512)
    sess = make_session(rg, model.export())
    want = sess.run(x)
    dx = rg.DeviceBuffer.from_array(x)
    dy = rg.DeviceBuffer(want.nbytes)
    for _ in range(3):
        shape = sess.run_device(dx, x.shape, dy)
    sess.synchronize()
    assert shape == want.shape
    assert_bitexact_f32(dy.download(want.shape), want)
    sess.set_capture(False)
    sess.set_profiling(0)
    sess.run_device(dx, x.shape, dy)
    sess.synchronize()
    assert_bitexact_f32(dy.download(want.shape), want)
    assert sess.last_npu_profile().total_time_ns > 0


def test_benchmark_regions(rg, ref):
    """The bench's timed regions (plain, with kernel events, with the
    memory-side cache displaced before each run) compute the same output as
    run(), and the event regions time every op."""
    from rustgears_amd import configs
    model, x = configs.deep_mlp(rows=512)
    sess = make_session(rg, model.export())
    want = sess.run(x)
    dx = rg.DeviceBuffer.from_array(x)
    dy = rg.DeviceBuffer(want.nbytes)
    for kw in ({"per_kernel_events": False}, {"per_kernel_events": True},
               {"per_kernel_events": True, "evict_cache": True}, {"per_kernel_events": False, "evict_cache": True}):
        print(f"[benchmark] {kw}", flush=True)
        ms, recs = sess.benchmark(dx, x.shape, dy, 3, **kw)
        assert ms > 0
        assert_bitexact_f32(dy.download(want.shape), want, str(kw))
        assert len(recs) == 3 and [r.op for r in recs] == [r.op for r in sess.last_npu_profile().records]
        if kw["per_kernel_events"]:
            assert all(r.duration_ns > 0 and r.kernel_ns > 0 for r in recs)
        dy.upload(np.zeros(want.shape, np.float32))


@pytest.mark.parametrize("kind", ["linear_small", "linear_large", "conv_first", "pool_first"])
def test_consecutive_runs_on_one_session(rg, ref, kind):
    """Several runs of one session with alternating input magnitudes: the
    absmax slots are reused run after run (double-buffered, cleared by each
    run's first kernel, or zero-filled), so a stale larger absmax would show
    up as a wrong scale in a later, smaller run."""
    from rustgears_amd import nn
    rg.manual_seed(23)
    if kind == "linear_small":  # GEMV path
        model = nn.Sequential().add(nn.Linear(512, 256)).add(nn.Tanh()).add(nn.Linear(256, 64))
        shape = [4, 512]
    elif kind == "linear_large":
        model = nn.Sequential().add(nn.Linear(300, 256)).add(nn.Relu()).add(nn.Linear(256, 32))
        shape = [700, 300]
    elif kind == "conv_first":
        model = (nn.Sequential().add(nn.Conv2d(3, 8, 3).padding(1)).add(nn.Relu()).add(nn.MaxPool2d(2))
                 .add(nn.Flatten()).add(nn.Linear(8 * 4 * 4, 10)))
        shape = [6, 3, 8, 8]
    else:  # first kernel is a max pool: the slots are zero-filled each run
        model = nn.Sequential().add(nn.MaxPool2d(2)).add(nn.Conv2d(3, 4, 3)).add(nn.Flatten()).add(nn.Linear(4 * 2 * 2, 5))
        shape = [5, 3, 8, 8]
    layers = model.export()
    sess = make_session(rg, layers)
    p = ref.RefProgram(layers)
    for i, mag in enumerate([50.0, 0.01, 3.0, 1e-3, 200.0]):
        print(f"[parity] consecutive {kind} run {i} magnitude {mag}", flush=True)
        x = (rg.randn(shape) * mag).astype(np.float32)
        assert_bitexact_f32(sess.run(x), p.run(x), f"{kind} run {i}")
    sess.close()


def _random_model(seed):
    """A seeded random layer stack: an optional conv section (1-2 convs with
    random channels, window 1/2/3/5, stride 1/2, padding 0-2, each optionally
    followed by a folding ChannelAffine, an activation and a max pool),
    Flatten, then 1-3 Linears with the same optional extras, an optional lone
    ChannelAffine at the start of the dense section and an optional Softmax."""
    from rustgears_amd.inference import Activation, LayerSpec
    g = np.random.default_rng(seed)
    acts = [Activation.RELU, Activation.SIGMOID, Activation.TANH, Activation.GELU, Activation.leaky_relu(0.2),
            Activation.SILU, Activation.NONE]
    f32 = lambda a: np.asarray(a, np.float32)
    layers = []
    if g.random() < 0.5:
        n, C, H, W = int(g.choice([1, 2, 5, 16])), int(g.integers(1, 20)), int(g.integers(4, 20)), int(g.integers(4, 20))
        shape = [n, C, H, W]
        for _ in range(int(g.integers(1, 3))):
            O, k, st, pd = int(g.integers(1, 48)), int(g.choice([1, 2, 3, 5])), int(g.choice([1, 2])), int(g.integers(0, 3))
            if H + 2 * pd < k or W + 2 * pd < k:
                k = 1
            layers.append(LayerSpec.Conv2d(C, O, k, st, pd, f32(g.standard_normal(O * C * k * k) / np.sqrt(C * k * k)),
                                           f32(g.standard_normal(O) * 0.1)))
            H, W, C = (H + 2 * pd - k) // st + 1, (W + 2 * pd - k) // st + 1, O
            if g.random() < 0.4:
                layers.append(LayerSpec.ChannelAffine(f32(g.uniform(0.5, 1.5, C)), f32(g.standard_normal(C) * 0.1)))
            if g.random() < 0.7:
                layers.append(LayerSpec.Activation(acts[int(g.integers(0, len(acts)))]))
            if g.random() < 0.5 and min(H, W) >= 2:
                pk = 3 if min(H, W) >= 3 and g.random() < 0.3 else 2
                ps = int(g.choice([1, 2]))
                layers.append(LayerSpec.MaxPool2d(pk, ps))
                H, W = (H - pk) // ps + 1, (W - pk) // ps + 1
        layers.append(LayerSpec.Flatten())
        F = C * H * W
    else:
        rows, F = int(g.choice([1, 3, 8, 9, 64, 300, 513])), int(g.integers(1, 700))
        shape = [rows, F]
        if g.random() < 0.2:
            layers.append(LayerSpec.ChannelAffine(f32(g.uniform(0.5, 1.5, F)), f32(g.standard_normal(F) * 0.1)))
    for _ in range(int(g.integers(1, 4))):
        out = int(g.choice([1, 3, 10, 16, 17, 64, 130, 300]))
        layers.append(LayerSpec.Linear(F, out, f32(g.standard_normal(F * out) / np.sqrt(F)), f32(g.standard_normal(out) * 0.1)))
        F = out
        if g.random() < 0.3:
            layers.append(LayerSpec.ChannelAffine(f32(g.uniform(0.5, 1.5, F)), f32(g.standard_normal(F) * 0.1)))
        if g.random() < 0.7:
            layers.append(LayerSpec.Activation(acts[int(g.integers(0, len(acts)))]))
    if g.random() < 0.3:
        layers.append(LayerSpec.Softmax())
    x = f32(g.standard_normal(shape) * float(g.choice([0.5, 1.0, 3.0])))
    return layers, x


@pytest.mark.parametrize("seed", range(64))
def test_random_models(rg, ref, seed):
    """Seeded random layer stacks through the whole plan (buffer ping-pong,
    slot layout, fusion and folding rules, every kernel choice): every op
    bit-exact with the oracle in capture mode, then the output of the
    production plan (no capture: the whole-program MLP, the small-tile GEMM
    quantizing as it loads, the fused requantization, the quantizing GEMVs and
    narrow heads, where the shapes take them) bit-exact with the same."""
    layers, x = _random_model(1000 + seed)
    what = f"random model {seed}: {[type(l).__name__ for l in layers]}"
    y = check_against_oracle(rg, ref, layers, x, what)
    print(f"[parity] {what} production plan", flush=True)
    sess = make_session(rg, layers)
    assert_bitexact_f32(sess.run(x), y, what + " production plan")
    sess.close()


def test_reference_integration_model(rg, ref):
    """The reference's own NPU integration test (integration.rs:127-164) on the
    MI355X provider: 9 raw layers fuse to 5 ops with the reference's labels,
    the weights compress more than 3x, the INT8 output stays within 0.15 of
    the fp32 model (BN statistics warmed by one training forward), and it is
    bit-exact with the oracle."""
    from test_oracle import _bn_eval, _bn_train_update, _np_conv
    from rustgears_amd import nn
    rg.manual_seed(2026)
    conv, bn2 = nn.Conv2d(1, 4, 3).padding(1), nn.BatchNorm2d(4)
    l1, bn1, l2 = nn.Linear(64, 16), nn.BatchNorm1d(16), nn.Linear(16, 4)
    model = (nn.Sequential().add(conv).add(bn2).add(nn.Relu()).add(nn.MaxPool2d(2)).add(nn.Flatten())
             .add(l1).add(bn1).add(nn.Relu()).add(l2))
    x = rg.randn([8, 1, 8, 8])
    xd = x.astype(np.float64)
    h = _np_conv(xd, conv.weight.astype(np.float64), conv.bias.astype(np.float64), 1)
    h = np.maximum(_bn_train_update(bn2, h), 0)
    h = h.reshape(8, 4, 4, 2, 4, 2).max(axis=(3, 5)).reshape(8, 64)
    _bn_train_update(bn1, h @ l1.weight + l1.bias)
    h = _np_conv(xd, conv.weight.astype(np.float64), conv.bias.astype(np.float64), 1)
    h = np.maximum(_bn_eval(bn2, h), 0)
    h = h.reshape(8, 4, 4, 2, 4, 2).max(axis=(3, 5)).reshape(8, 64)
    fp32 = np.maximum(_bn_eval(bn1, h @ l1.weight + l1.bias), 0) @ l2.weight + l2.bias
    layers = model.export()
    y = check_against_oracle(rg, ref, layers, x, "integration.rs model")
    sess = make_session(rg, layers)
    sess.run(x)
    prof = sess.last_npu_profile()
    assert prof.original_layers == 9 and prof.fused_ops == 5
    assert prof.compression_ratio() > 3.0
    assert [r.op for r in prof.records] == ["NPU::FusedConv2dAct(1->4, k=3, ReLU)", "NPU::MaxPool2d(k=2)",
                                            "NPU::Flatten", "NPU::FusedGemmAct(64->16, ReLU)", "NPU::Gemm(16->4)"]
    assert np.abs(y - fp32).max() <= 0.15
    sess.close()


def test_compilation_report(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(0)
    model = nn.Sequential().add(nn.Linear(16, 64)).add(nn.BatchNorm1d(64)).add(nn.Relu()).add(nn.Linear(64, 4))
    sess = rg.InferenceSession.from_module(model, rg.ExecutionProvider.mi355x_int8())
    assert sess.compilation_report() == (
        "InferenceSession [provider = MI355X (INT8), layers: 4 -> 2 fused ops, weights: 5392 B -> 1560 B "
        "(3.46x compression)]\n  Pipeline: NPU::FusedGemmAct(16->64, ReLU) -> NPU::Gemm(64->4)")
    sess.run(rg.randn([32, 16]))
    prof = sess.last_npu_profile()
    assert prof.total_macs == 40960 and prof.compression_ratio() > 3.0
