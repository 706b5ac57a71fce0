"""Certified GELU requantization (requant.hip, rgmath::gelu_approx).

A Linear + GELU whose output only feeds the next Linear's quantization
(npu.rs:312, quantize.rs:18-24) hands on two things: the tensor's absmax and
every value's quantized integer.  The fused GEMM gets both exactly without
the exact GELU on every value: the absmax from each lane's largest
pre-activation (the f32 GELU never decreases on [0, +inf] and stays within
kGeluNegAbsMax below 0), the integers from gelu_approx within its certified
bound, with the exact GELU where the bound cannot decide.  These tests check
the results bit for bit against the oracle:

* every tile shape of the fused GEMM in the modes of RGNPU_GELU_CERT:
  1 certified; 3 certified with a margin that sends a few values in a
  thousand through the per-wave LDS queue of exact fallbacks; 2 every value
  uncertain (each queue overflows: the exact re-walk); 0 the exact GELU
  everywhere.  Also with deferral to the finisher;
* tensors whose absmax comes from negative pre-activations (no lane clears
  the bound, so every workgroup takes the exact absmax walk), and a mix of
  workgroups that do and do not;
* NaN and -inf pre-activations (bias columns), whose GELU is NaN: ignored by
  the absmax, quantized to 0.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def _gelu_chain(rg, dims, seed):
    from rustgears_amd import nn
    rg.manual_seed(seed)
    m = nn.Sequential()
    for a, b in zip(dims[:-1], dims[1:]):
        m.add(nn.Linear(a, b)).add(nn.Gelu())
    return m.export()


def _run_modes(rg, ref, monkeypatch, layers, x, what, modes=("1", "3", "2", "0"), spin=None):
    want = ref.RefProgram(layers).run(x, parallel=True)
    if spin is not None:
        monkeypatch.setenv("RGNPU_REQUANT_SPIN_LIMIT", spin)
    for mode in modes:
        monkeypatch.setenv("RGNPU_GELU_CERT", mode)
        print(f"[gelu-cert] {what} x{tuple(x.shape)} mode {mode} spin {spin}", flush=True)
        sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
        y = sess.run(x)
        y2 = sess.run(x)
        prof = sess.last_npu_profile()
        sess.close()
        assert_bitexact_f32(y, want, f"{what} mode {mode}")
        assert_bitexact_f32(y2, want, f"{what} mode {mode} (second run)")
        # the second Linear's input was quantized by its producer (fused path)
        gemms = [r for r in prof.records if "Gemm" in r.op]
        assert gemms[1].duration_ns == gemms[1].kernel_ns, gemms


CHAINS = [
    # (name, dims, rows): the tile shape of the fused GEMMs
    ("256x256 multi-tile", [4000, 4000, 4000], 4400),  # 18 x 16 = 288 tiles: two per workgroup for some
    ("256x128", [1000, 3000, 2000, 500], 2600),
    ("128x128 ragged", [700, 2004, 1516], 1500),
    ("four fused", [256, 384, 512, 384, 132], 2048),
]


@pytest.mark.parametrize("name,dims,rows", CHAINS, ids=[c[0] for c in CHAINS])
def test_certified_gelu_modes(rg, ref, monkeypatch, name, dims, rows):
    layers = _gelu_chain(rg, dims, seed=rows + 7)
    x = rg.randn([rows, dims[0]])
    _run_modes(rg, ref, monkeypatch, layers, x, name)


def test_certified_gelu_deferred(rg, ref, monkeypatch):
    """No workgroup waits at the barrier: the finisher quantizes every other
    workgroup's tiles from their stored pre-activations."""
    layers = _gelu_chain(rg, [4000, 4000, 4000], seed=4407)
    x = rg.randn([4400, 4000])
    _run_modes(rg, ref, monkeypatch, layers, x, "256x256 deferred", modes=("1", "3", "2"), spin="0")


def _small_negative(rg, seed, n_hot):
    """Linear(512, 1024) + GELU -> Linear(1024, 64) + GELU with tiny weights
    and biases near -0.75 (the GELU minimum): pre-activations in about
    [-0.8, -0.7], so the absmax (~0.17) comes from negative values.  n_hot
    columns get a bias of +2, so their lanes see large positive values."""
    layers = _gelu_chain(rg, [512, 1024, 64], seed=seed)
    lin = layers[0]
    lin.weight = (lin.weight * np.float32(1e-3)).astype(np.float32)
    gen = np.random.default_rng(seed)
    lin.bias = (np.float32(-0.75) + gen.uniform(-0.04, 0.04, lin.bias.shape)).astype(np.float32)
    if n_hot:
        lin.bias[gen.choice(lin.bias.size, n_hot, replace=False)] = np.float32(2.0)
    return layers


@pytest.mark.parametrize("n_hot", [0, 3], ids=["all-negative", "three-hot-columns"])
def test_certified_gelu_absmax_from_negative_values(rg, ref, monkeypatch, n_hot):
    layers = _small_negative(rg, 91 + n_hot, n_hot)
    x = rg.randn([2048, 512])
    _run_modes(rg, ref, monkeypatch, layers, x, f"negative pre-activations, {n_hot} hot", modes=("1", "3", "2"))


def test_certified_gelu_nan_and_neg_inf_preactivations(rg, ref, monkeypatch):
    """Bias columns of NaN and -inf: gelu(NaN) and gelu(-inf) = -inf * 0 are
    NaN, which f32::max ignores and the quantizer maps to 0."""
    layers = _gelu_chain(rg, [512, 1024, 64], seed=57)
    lin = layers[0]
    lin.bias[[3, 100, 513]] = np.float32(np.nan)
    lin.bias[[7, 900]] = np.float32(-np.inf)
    x = rg.randn([2048, 512])
    _run_modes(rg, ref, monkeypatch, layers, x, "NaN / -inf bias columns", modes=("1", "3", "2"))
