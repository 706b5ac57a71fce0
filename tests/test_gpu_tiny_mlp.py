"""Small INT8 Linear programs as one kernel (mlp_tiny_kernel).

A program whose every op is an INT8 Linear on the same rows (at most 64 rows,
128 features and Kpad, 8 layers, 48 KiB of weights) runs as one launch of one
workgroup: per layer its input's absmax, the quantization into LDS, the exact
i32 sums and the fused epilogue (npu.rs:307-318, quantize.rs:18-24, 93-118).
Each case is compared bit for bit with the oracle and with the per-op kernels
(RGNPU_TINY_MLP=0) on the same input: the quickstart program, chains over
every activation code with ragged widths and 1..64 rows, folded BatchNorm,
special input values, and programs on both sides of each limit.  The profile
keeps every op's record; the first holds the kernel's time and the others
report 0 ns.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def _program(rg, dims, acts, seed, bn_at=()):
    from rustgears_amd import configs, nn
    from rustgears_amd.inference import Activation, LayerSpec
    rg.manual_seed(seed)
    parts, bns = [], []
    mods = {"relu": nn.Relu, "sigmoid": nn.Sigmoid, "tanh": nn.Tanh, "gelu": nn.Gelu}
    for i in range(len(dims) - 1):
        parts.append(nn.Linear(dims[i], dims[i + 1]))
        if i in bn_at:
            bn = nn.BatchNorm1d(dims[i + 1])
            bns.append(bn)
            parts.append(bn)
        a = acts[i % len(acts)]
        if a == "silu":
            parts.append([LayerSpec.Activation(Activation.SILU)])
        elif a == "leaky":
            parts.append(nn.LeakyRelu(0.03))
        elif a is not None:
            parts.append(mods[a]())
    configs.set_bn_stats(bns)
    layers = []
    for p in parts:
        layers += p if isinstance(p, list) else p.export()
    return layers


def _run(rg, layers, x, tiny, monkeypatch):
    if tiny:
        monkeypatch.delenv("RGNPU_TINY_MLP", raising=False)
    else:
        monkeypatch.setenv("RGNPU_TINY_MLP", "0")
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    y2 = sess.run(x)
    recs = list(sess.last_npu_profile().records)
    sess.close()
    monkeypatch.delenv("RGNPU_TINY_MLP", raising=False)
    assert_bitexact_f32(y2, y, "second run")
    return y, recs


def _check(rg, ref, monkeypatch, layers, x, what, expect_tiny=True):
    print(f"[tiny] {what} x{tuple(x.shape)}", flush=True)
    want = ref.RefProgram(layers).run(x, parallel=True)
    y, recs = _run(rg, layers, x, True, monkeypatch)
    y0, recs0 = _run(rg, layers, x, False, monkeypatch)
    assert_bitexact_f32(y, want, what + " (one kernel) vs oracle")
    assert_bitexact_f32(y0, want, what + " (per-op kernels) vs oracle")
    assert [r.op for r in recs] == [r.op for r in recs0] and [r.macs for r in recs] == [r.macs for r in recs0]
    if expect_tiny:
        assert recs[0].kernel_ns > 0, recs[0]
        assert all(r.duration_ns == 0 and r.kernel_ns == 0 for r in recs[1:]), recs
    else:
        assert all(r.kernel_ns > 0 for r in recs), recs
    assert all(r.kernel_ns > 0 for r in recs0), recs0
    return recs


def test_quickstart_runs_as_one_kernel(rg, ref, monkeypatch):
    from rustgears_amd import configs
    model, x = configs.quickstart()
    recs = _check(rg, ref, monkeypatch, model.export(), x, "quickstart")
    assert [r.op for r in recs] == ["NPU::FusedGemmAct(4->32, ReLU)", "NPU::Gemm(32->3)"]


CASES = [
    # (name, dims, acts, rows, bn_at)
    ("one layer", [16, 8], [None], 64, ()),
    ("gelu silu none", [32, 128, 64, 10], ["gelu", "silu", None], 64, ()),
    ("every activation, 8 layers", [7, 33, 17, 100, 5, 128, 3, 64, 9],
     ["relu", "sigmoid", "tanh", "gelu", "leaky", "silu", None, "relu"], 37, ()),
    ("one row", [64, 128, 128], ["gelu"], 1, ()),
    ("63 rows leaky", [128, 128, 128, 128], ["leaky"], 63, ()),
    ("folded batch norm", [4, 32, 16, 3], ["relu", "tanh"], 64, (0, 1)),
    ("weights at the limit", [128, 128, 128, 128], ["sigmoid"], 64, ()),
    ("width 1", [1, 1, 5, 1], ["tanh", None], 9, ()),
]


@pytest.mark.parametrize("name,dims,acts,rows,bn_at", CASES, ids=[c[0] for c in CASES])
def test_chain_matches_oracle_and_per_op_kernels(rg, ref, monkeypatch, name, dims, acts, rows, bn_at):
    layers = _program(rg, dims, acts, seed=len(dims) * 100 + rows, bn_at=bn_at)
    x = rg.randn([rows, dims[0]]) * np.float32(3.0)
    _check(rg, ref, monkeypatch, layers, x, name)


BEYOND = [
    # one limit exceeded each: the per-op kernels run
    ("65 rows", [32, 32, 8], ["relu"], 65),
    ("129 features", [32, 129, 8], ["relu"], 64),
    ("9 layers", [8] * 10, ["relu"], 16),
    ("64 KiB of weights", [128, 128, 128, 128, 128], ["relu"], 16),
]


@pytest.mark.parametrize("name,dims,acts,rows", BEYOND, ids=[c[0] for c in BEYOND])
def test_programs_past_a_limit_use_the_per_op_kernels(rg, ref, monkeypatch, name, dims, acts, rows):
    layers = _program(rg, dims, acts, seed=rows + 7)
    _check(rg, ref, monkeypatch, layers, rg.randn([rows, dims[0]]), name, expect_tiny=False)


def test_programs_with_other_ops_use_the_per_op_kernels(rg, ref, monkeypatch):
    """A second activation after a fused one stays an op of its own, so the
    program is more than a chain of Linears."""
    from rustgears_amd import nn
    from rustgears_amd.inference import Activation, LayerSpec
    rg.manual_seed(31)
    layers = (nn.Sequential().add(nn.Linear(16, 32)).add(nn.Relu()).export() +
              [LayerSpec.Activation(Activation.TANH)] + nn.Linear(32, 4).export())
    _check(rg, ref, monkeypatch, layers, rg.randn([32, 16]), "lone activation", expect_tiny=False)


def test_special_input_values(rg, ref, monkeypatch):
    """NaN (ignored by the absmax, quantized to 0), infinities (the scale
    becomes infinite and every finite value quantizes to 0), signed zeros,
    subnormals and an all-zero tensor (scale 1)."""
    layers = _program(rg, [8, 24, 6], ["gelu", None], seed=5)
    base = rg.randn([16, 8])
    specials = np.array([np.nan, -np.nan, 0.0, -0.0, 1e-40, -1e-45, 3e38, -3e38], np.float32)
    x = base.copy()
    x[0] = specials
    x[3, ::2] = np.nan
    _check(rg, ref, monkeypatch, layers, x, "NaN, subnormals, large")
    xi = base.copy()
    xi[5, 1] = np.inf
    xi[7, 2] = -np.inf
    _check(rg, ref, monkeypatch, layers, xi, "infinities")
    _check(rg, ref, monkeypatch, layers, np.zeros([16, 8], np.float32), "all zeros")


def test_consecutive_runs_reuse_the_slots(rg, ref):
    """Alternating input magnitudes on one session: each run's absmax slots
    are the set its first (and only) kernel did not clear."""
    layers = _program(rg, [16, 64, 64, 8], ["relu", "gelu"], seed=11)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    prog = ref.RefProgram(layers)
    for k in range(6):
        x = rg.randn([48, 16]) * np.float32(10.0 ** (3 * (k % 2) - 1))
        assert_bitexact_f32(sess.run(x), prog.run(x), f"run {k}")
    sess.close()


def test_production_taps_on_one_kernel(rg, ref):
    """Production taps on the one-kernel program: every op's scale comes from
    the absmax key the kernel writes into the op's slot; the i8 operands and
    the first op's f32 output live only in LDS, so only the last op's output
    is tapped."""
    from rustgears_amd import configs
    model, x = configs.quickstart()
    layers = model.export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    sess.set_capture("production")
    y = sess.run(x)
    prog = ref.RefProgram(layers)
    prog.set_capture(True)
    yr = prog.run(x)
    for i in range(prog.num_ops):
        assert sess.capture(i, 0).size == 0, i
        assert_bitexact_f32(sess.capture(i, 1), prog.capture(i, 1), f"op{i} scale")
    assert sess.capture(0, 3).size == 0
    assert_bitexact_f32(sess.capture(1, 3), prog.capture(1, 3), "op1 out")
    assert_bitexact_f32(y, yr, "output")
    sess.close()
