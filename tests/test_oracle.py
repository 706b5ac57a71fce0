"""Pins for the CPU oracle (oracle/rgref.c).

The reference is Rust and cannot be built here (no rustc/cargo), so the
oracle is a C restatement.  Each test below checks one oracle function
against something independent of the restated formula: a published vector,
a closed form, brute force in numpy, or the reference's own tests
(integration.rs:127-164, vision.rs:102-109, USAGE.md:377-381).
"""
import ctypes
import math
import os

import numpy as np
import pytest

from conftest import assert_bitexact_f32, quantize_np, round_half_away


# ---- rng.rs ---------------------------------------------------------------------
def test_splitmix64_published_vector(ref):
    # Vigna's splitmix64.c from state 0: Rng::new(seed) stores seed ^ gamma,
    # so seed = gamma gives state 0 (rng.rs:16-18).
    r = ref.RefRng()
    ref.lib().rgref_rng_new(r, 0x9E3779B97F4A7C15)
    got = [ref.lib().rgref_rng_next_u64(r) for _ in range(3)]
    assert got == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def _splitmix_py(seed, n):
    mask = (1 << 64) - 1
    state = seed ^ 0x9E3779B97F4A7C15
    out = []
    for _ in range(n):
        state = (state + 0x9E3779B97F4A7C15) & mask
        z = state
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & mask
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & mask
        out.append(z ^ (z >> 31))
    return out


def test_uniform_closed_form(ref):
    # uniform = (u64 >> 40) / 2^24 exactly (rng.rs:30-32); checked against a
    # Python big-int SplitMix64 for several seeds.
    for seed in (0, 1, 42, 0x5EED, 2**63 + 5):
        ref.manual_seed(seed)
        got = ref.fill("uniform", [257])
        want = np.array([(u >> 40) / float(1 << 24) for u in _splitmix_py(seed, 257)], np.float32)
        assert_bitexact_f32(got, want, f"seed {seed}")


def test_uniform_range_closed_form(ref):
    ref.manual_seed(9)
    u = ref.fill("uniform", [1000])
    ref.manual_seed(9)
    got = ref.fill("range", [1000], -0.25, 0.75)
    want = (np.float32(-0.25) + (np.float32(0.75) - np.float32(-0.25)) * u).astype(np.float32)
    assert_bitexact_f32(got, want)


def test_normal_box_muller(ref):
    # randn consumes two uniforms per sample: u1 clamped to 1e-7, then u2
    # (rng.rs:40-44).  Compared with the formula in double precision; a
    # swapped u1/u2, missing 2*pi or wrong clamp breaks this by far more.
    ref.manual_seed(123)
    u = ref.fill("uniform", [20000]).astype(np.float64)
    ref.manual_seed(123)
    z = ref.fill("normal", [10000]).astype(np.float64)
    u1 = np.maximum(u[0::2], 1e-7)
    u2 = u[1::2]
    want = np.sqrt(-2.0 * np.log(u1)) * np.cos(2.0 * np.pi * u2)
    assert np.allclose(z, want, rtol=2e-5, atol=2e-6)
    assert abs(z.mean()) < 0.05 and abs(z.std() - 1.0) < 0.05


def test_default_global_seed_is_5eed(ref):
    # A fresh global generator uses 0x5EED (rng.rs:66); manual_seed(0x5EED)
    # must reproduce the same stream.
    ref.manual_seed(0x5EED)
    a = ref.fill("uniform", [8])
    want = np.array([(u >> 40) / float(1 << 24) for u in _splitmix_py(0x5EED, 8)], np.float32)
    assert_bitexact_f32(a, want)


# ---- quantize.rs ------------------------------------------------------------------
def test_quantize_closed_forms(ref):
    # absmax 127 -> scale 1, inv 1: q = round half away from zero.
    v = np.array([127.0, -127.0, 2.5, -2.5, 0.5, -0.5, 1.49999988, -1.5, 0.0, -0.0, 126.5], np.float32)
    q, s = ref.quantize(v)
    assert s == np.float32(1.0)
    assert q.tolist() == [127, -127, 3, -3, 1, -1, 1, -2, 0, 0, 127]


def test_quantize_scale_rule(ref):
    v = np.array([0.3, -2.54, 1.0], np.float32)
    q, s = ref.quantize(v)
    assert s == np.float32(np.float32(2.54) / np.float32(127.0))
    assert q.tolist() == [15, -127, 50]
    # max_abs < 1e-12 -> scale 1 and everything rounds to 0
    q, s = ref.quantize(np.array([1e-13, -5e-13, 0.0], np.float32))
    assert s == np.float32(1.0) and q.tolist() == [0, 0, 0]
    # all zeros
    q, s = ref.quantize(np.zeros(5, np.float32))
    assert s == np.float32(1.0) and not q.any()


def test_quantize_nan_inf(ref):
    # f32::max ignores NaN; NaN quantizes to 0 (`as i8`).
    q, s = ref.quantize(np.array([np.nan, 1.27, -0.635], np.float32))
    assert s == np.float32(np.float32(1.27) / np.float32(127.0))
    assert q.tolist() == [0, 127, -64]
    # +-Inf: scale = Inf, inv = 0, finite*0 = 0, Inf*0 = NaN -> 0
    q, s = ref.quantize(np.array([np.inf, 3.0, -np.inf], np.float32))
    assert np.isinf(s) and q.tolist() == [0, 0, 0]
    # all NaN -> max_abs 0 -> scale 1
    q, s = ref.quantize(np.array([np.nan, np.nan], np.float32))
    assert s == np.float32(1.0) and q.tolist() == [0, 0]


def test_quantize_random_vs_numpy(ref):
    rng = np.random.default_rng(0)
    for n in (1, 7, 1000, 4099):
        v = (rng.standard_normal(n) * rng.uniform(0.01, 100)).astype(np.float32)
        q, s = ref.quantize(v)
        q2, s2 = quantize_np(v)
        assert s == s2 and np.array_equal(q, q2)
        assert q.min() >= -127 and q.max() <= 127


# ---- dot_i8 / GEMM ---------------------------------------------------------------
@pytest.mark.parametrize("m,k,n", [(1, 1, 1), (3, 5, 7), (8, 27, 32), (17, 288, 9), (64, 1024, 40)])
def test_gemm_accumulators_brute_force(ref, m, k, n):
    rng = np.random.default_rng(m * 1000 + k)
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    bias = rng.standard_normal(n).astype(np.float32)
    out, acc = ref.gemm_fused(a, np.float32(0.01), b, np.float32(0.02), m, k, n, bias)
    want = a.astype(np.int64) @ b.astype(np.int64).T
    assert np.array_equal(acc, want.astype(np.int32))
    # epilogue closed form fl(fl(fl(acc) * fl(sa*sw)) + b), act None
    cs = np.float32(np.float32(0.01) * np.float32(0.02))
    want_out = ((acc.astype(np.float32) * cs).astype(np.float32) + bias).astype(np.float32)
    assert_bitexact_f32(out, want_out)


def test_gemm_parallel_equals_serial(ref):
    rng = np.random.default_rng(3)
    m, k, n = 64, 256, 48
    a = rng.integers(-127, 128, (m, k), dtype=np.int8)
    b = rng.integers(-127, 128, (n, k), dtype=np.int8)
    bias = rng.standard_normal(n).astype(np.float32)
    o1, a1 = ref.gemm_fused(a, 0.5, b, 0.25, m, k, n, bias, act=1, parallel=False)
    o2, a2 = ref.gemm_fused(a, 0.5, b, 0.25, m, k, n, bias, act=1, parallel=True)
    assert np.array_equal(a1, a2)
    assert_bitexact_f32(o1, o2)


# ---- activations (backend.rs:66-78) -----------------------------------------------
def test_relu_leaky_closed_forms(ref):
    x = np.array([-3.0, -0.0, 0.0, 2.5, np.nan, -np.inf, np.inf], np.float32)
    r = ref.act_apply(1, 0.0, x)
    assert r[0] == 0 and r[3] == 2.5 and r[4] == 0 and r[5] == 0 and r[6] == np.inf  # NaN.max(0) = 0
    # Sign of zero: ReLU(-0.0) is +0.0 (see test_relu_matches_llvm_maxnum_lowering).
    bits = r.view(np.uint32)
    assert bits[1] == 0 and bits[2] == 0 and bits[0] == 0 and bits[4] == 0 and bits[5] == 0
    lr = ref.act_apply(5, 0.1, x)
    assert lr[0] == np.float32(np.float32(0.1) * np.float32(-3.0)) and lr[3] == 2.5


def test_relu_matches_llvm_maxnum_lowering(ref, tmp_path):
    """ReLU is x.max(0.0) (backend.rs:71): Rust lowers f32::max to
    llvm.maxnum, whose sign of an equal-zero result is left to the backend.
    clang lowers fmaxf to the same intrinsic, so a function compiled by the
    LLVM x86-64 backend shows the bits the reference's build produces: the
    oracle must agree on signed zeros, NaN, infinities and denormals."""
    import shutil
    import subprocess
    clang = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "llvm", "bin", "clang")
    if not os.path.exists(clang):
        clang = shutil.which("clang")
    if not clang:
        pytest.skip("no LLVM clang for the host")
    src = tmp_path / "relu.c"
    src.write_text("float relu(float x) { return __builtin_fmaxf(x, 0.0f); }\n")
    ir = subprocess.run([clang, "-O2", "-S", "-emit-llvm", "-o", "-", str(src)], capture_output=True, text=True)
    assert "llvm.maxnum.f32" in ir.stdout, "fmaxf must lower to llvm.maxnum, as f32::max does"
    so = tmp_path / "librelu.so"
    subprocess.run([clang, "-O2", "-shared", "-fPIC", "-o", str(so), str(src)], check=True)
    lib = ctypes.CDLL(str(so))
    lib.relu.restype, lib.relu.argtypes = ctypes.c_float, [ctypes.c_float]
    x = np.array([-0.0, 0.0, -1.0, 1.0, np.nan, -np.inf, np.inf, 1e-45, -1e-45, 3.5e38, -2.5], np.float32)
    want = np.array([lib.relu(float(v)) for v in x], np.float32)
    got = ref.act_apply(1, 0.0, x)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), (got, want)
    assert want.view(np.uint32)[0] == 0  # -0.0 -> +0.0


def test_transcendental_activations_near_exact(ref):
    # GELU / Sigmoid / Tanh / SiLU use host libm tanhf/expf.  Pinned against
    # double-precision evaluation of the same expressions (<= a few ulp) and
    # special values; a wrong constant (GELU_C, 0.044715) or a dropped term
    # would miss by orders of magnitude more.
    rng = np.random.default_rng(5)
    x = np.concatenate([rng.standard_normal(4000) * 4, np.linspace(-20, 20, 801)]).astype(np.float32)
    xd = x.astype(np.float64)
    tanh = ref.act_apply(3, 0.0, x)
    assert np.allclose(tanh, np.tanh(xd), rtol=3e-7, atol=1e-30)
    sig = ref.act_apply(2, 0.0, x)
    assert np.allclose(sig, 1 / (1 + np.exp(-xd)), rtol=1e-6)
    gelu = ref.act_apply(4, 0.0, x)
    c = np.float64(np.float32(0.7978846))
    want = 0.5 * xd * (1 + np.tanh(c * (xd + np.float64(np.float32(0.044715)) * xd ** 3)))
    assert np.allclose(gelu, want, rtol=2e-6, atol=1e-6)
    silu = ref.act_apply(6, 0.0, x)
    assert np.allclose(silu, xd / (1 + np.exp(-xd)), rtol=2e-6, atol=1e-7)
    sp = ref.act_apply(3, 0.0, np.array([0.0, np.inf, -np.inf, 30.0], np.float32))
    assert sp.tolist() == [0.0, 1.0, -1.0, 1.0]
    assert ref.act_apply(2, 0.0, np.array([0.0], np.float32))[0] == np.float32(0.5)
    assert ref.act_apply(4, 0.0, np.array([0.0], np.float32))[0] == 0.0


# ---- kernels.rs / shape.rs ----------------------------------------------------------
def _im2col_brute(x, c, h, w, k, s, p):
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    cols = np.zeros((c * k * k, oh * ow), np.float32)
    for ch in range(c):
        for ki in range(k):
            for kj in range(k):
                for oy in range(oh):
                    for ox in range(ow):
                        iy, ix = oy * s + ki - p, ox * s + kj - p
                        if 0 <= iy < h and 0 <= ix < w:
                            cols[(ch * k + ki) * k + kj, oy * ow + ox] = x[ch, iy, ix]
    return cols


@pytest.mark.parametrize("c,h,w,k,s,p", [(3, 8, 8, 3, 1, 1), (2, 7, 5, 3, 2, 0), (1, 6, 6, 1, 3, 0),
                                         (4, 5, 9, 2, 1, 2), (2, 9, 9, 2, 3, 1)])
def test_im2col_brute_force(ref, c, h, w, k, s, p):
    x = np.random.default_rng(c * h).standard_normal((c, h, w)).astype(np.float32)
    assert_bitexact_f32(ref.im2col(x, c, h, w, k, s, p), _im2col_brute(x, c, h, w, k, s, p))


def test_out_size_rules(ref):
    o = ref.lib().rgref_out_size
    assert o(32, 3, 1, 1) == 32 and o(32, 2, 2, 0) == 16 and o(5, 2, 2, 0) == 2
    assert o(2, 5, 1, 0) == -1  # kernel larger than padded input (kernels.rs:13 panics)


def test_max_pool_brute_force_and_nan_rules(ref):
    x = np.random.default_rng(1).standard_normal((2, 3, 7, 6)).astype(np.float32)
    got = ref.max_pool2d(x, 2, 3, 7, 6, 2, 2)
    want = np.zeros((2, 3, 3, 3), np.float32)
    for i in range(3):
        for j in range(3):
            want[:, :, i, j] = x[:, :, 2 * i:2 * i + 2, 2 * j:2 * j + 2].max(axis=(2, 3))
    assert_bitexact_f32(got, want)
    # vision.rs:102-109: -inf windows stay -inf, NaN propagates
    ninf = np.full((2, 2, 2, 2), -np.inf, np.float32)
    assert np.all(ref.max_pool2d(ninf, 2, 2, 2, 2, 1, 1) == -np.inf)
    nan = np.array([np.nan, 1.0], np.float32).reshape(1, 1, 1, 2)
    assert np.isnan(ref.max_pool2d(nan, 1, 1, 1, 2, 1, 1)[0, 0, 0, 0])
    win = np.array([1.0, np.nan, 5.0, 2.0], np.float32).reshape(1, 1, 2, 2)
    assert np.isnan(ref.max_pool2d(win, 1, 1, 2, 2, 2, 2)[0, 0, 0, 0])
    # kernels.rs:187: `v > best || v.is_nan()` -- a later NaN replaces an earlier
    # one (payload of the last NaN wins), and equal values keep the first, so
    # a (-0.0, +0.0) window gives -0.0 and (+0.0, -0.0) gives +0.0.
    nan2 = np.array([0x7fc00001, 0x7fc00002, 0, 0], np.uint32).view(np.float32).reshape(1, 1, 2, 2)
    assert ref.max_pool2d(nan2, 1, 1, 2, 2, 2, 2).view(np.uint32)[0, 0, 0, 0] == 0x7fc00002
    zz = np.array([-0.0, 0.0, 0.0, -0.0, -1, -1, -1, -1], np.float32).reshape(1, 1, 2, 4)
    assert ref.max_pool2d(zz, 1, 1, 2, 4, 2, 2).view(np.uint32).tolist() == [[[[0x80000000, 0]]]]


def test_softmax_rows(ref):
    x = np.random.default_rng(2).standard_normal((5, 11)).astype(np.float32)
    y = ref.softmax_rows(x)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    assert np.allclose(y, e / e.sum(axis=1, keepdims=True), rtol=1e-6)


# ---- compile / execute (npu.rs) ---------------------------------------------------
def test_usage_md_pipeline_example(ref, rg):
    # USAGE.md:366-381: Linear(16,64)+BN1d+ReLU+Linear(64,4), batch 32 ->
    # 2 fused ops, 40,960 MACs, 5392 fp32 weight bytes.  The doc's 1552 B is
    # stale; quantize.rs:43-45 adds a 4-byte scale per tensor: 1560 B.
    from rustgears_amd import nn
    rg.manual_seed(0)
    model = nn.Sequential().add(nn.Linear(16, 64)).add(nn.BatchNorm1d(64)).add(nn.Relu()).add(nn.Linear(64, 4))
    p = ref.RefProgram(model.export())
    assert p.labels() == ["NPU::FusedGemmAct(16->64, ReLU)", "NPU::Gemm(64->4)"]
    assert p.fp32_bytes == 5392 and p.npu_bytes == 1560 and p.original_layers == 4
    p.run(rg.randn([32, 16]))
    assert p.total_macs == 40960 and [p.op_macs(0), p.op_macs(1)] == [32768, 8192]


def _np_conv(x, w, b, pad):
    n, c, h, ww = x.shape
    o, _, k, _ = w.shape
    xp = np.pad(x, ((0, 0), (0, 0), (pad, pad), (pad, pad)))
    oh, ow = h + 2 * pad - k + 1, ww + 2 * pad - k + 1
    out = np.zeros((n, o, oh, ow), np.float64)
    for ki in range(k):
        for kj in range(k):
            patch = xp[:, :, ki:ki + oh, kj:kj + ow]
            out += np.einsum("nchw,oc->nohw", patch, w[:, :, ki, kj])
    return out + b[None, :, None, None]


def _bn_train_update(bn, x):
    axes = (0, 2, 3) if x.ndim == 4 else (0,)
    m = x.size // x.shape[1]
    mean = x.mean(axis=axes)
    var = x.var(axis=axes)
    bn.running_mean = (0.9 * bn.running_mean + 0.1 * mean).astype(np.float32)
    bn.running_var = (0.9 * bn.running_var + 0.1 * var * (m / (m - 1))).astype(np.float32)
    shape = (1, -1, 1, 1) if x.ndim == 4 else (1, -1)
    return (x - mean.reshape(shape)) / np.sqrt(var.reshape(shape) + 1e-5)


def _bn_eval(bn, x):
    shape = (1, -1, 1, 1) if x.ndim == 4 else (1, -1)
    return (x - bn.running_mean.reshape(shape)) / np.sqrt(bn.running_var.reshape(shape) + 1e-5)


def test_reference_integration_npu_fusion(ref, rg):
    # integration.rs:127-164: 9 raw layers -> 5 fused ops, compression > 3,
    # |int8 - fp32| <= 0.15 against the fp32 model after one BN-warming
    # training forward on randn[8,1,8,8].
    from rustgears_amd import nn
    rg.manual_seed(2026)
    conv, bn2 = nn.Conv2d(1, 4, 3).padding(1), nn.BatchNorm2d(4)
    l1, bn1, l2 = nn.Linear(64, 16), nn.BatchNorm1d(16), nn.Linear(16, 4)
    model = (nn.Sequential().add(conv).add(bn2).add(nn.Relu()).add(nn.MaxPool2d(2)).add(nn.Flatten())
             .add(l1).add(bn1).add(nn.Relu()).add(l2))
    x = rg.randn([8, 1, 8, 8])
    xd = x.astype(np.float64)
    # training forward (BN uses batch statistics and updates running stats)
    h = _np_conv(xd, conv.weight.astype(np.float64), conv.bias.astype(np.float64), 1)
    h = np.maximum(_bn_train_update(bn2, h), 0)
    h = h.reshape(8, 4, 4, 2, 4, 2).max(axis=(3, 5)).reshape(8, 64)
    h = h @ l1.weight + l1.bias
    _bn_train_update(bn1, h)
    # eval forward
    h = _np_conv(xd, conv.weight.astype(np.float64), conv.bias.astype(np.float64), 1)
    h = np.maximum(_bn_eval(bn2, h), 0)
    h = h.reshape(8, 4, 4, 2, 4, 2).max(axis=(3, 5)).reshape(8, 64)
    h = np.maximum(_bn_eval(bn1, h @ l1.weight + l1.bias), 0)
    fp32 = h @ l2.weight + l2.bias
    p = ref.RefProgram(model.export())
    assert p.original_layers == 9 and p.num_ops == 5
    assert p.fp32_bytes / p.npu_bytes > 3.0
    assert p.labels() == ["NPU::FusedConv2dAct(1->4, k=3, ReLU)", "NPU::MaxPool2d(k=2)", "NPU::Flatten",
                          "NPU::FusedGemmAct(64->16, ReLU)", "NPU::Gemm(16->4)"]
    out = p.run(x)
    assert np.abs(out - fp32).max() <= 0.15


def test_fold_batch_norm_and_weight_quantization(ref, rg):
    # fold_batch_norm (mod.rs:225-257) then transpose + per-tensor quantize
    # (npu.rs:208-209), recomputed in numpy.
    from rustgears_amd import nn
    rg.manual_seed(77)
    lin, bn = nn.Linear(6, 5), nn.BatchNorm1d(5)
    bn.running_mean = rg.randn([5])
    bn.running_var = rg.uniform([5], 0.5, 1.5)
    bn.gamma = rg.uniform([5], 0.5, 2.0)
    layers = nn.Sequential().add(lin).add(bn).add(nn.Relu()).export()
    aff = layers[1]
    w = (lin.weight * aff.scale[None, :]).astype(np.float32)
    b = ((lin.bias * aff.scale).astype(np.float32) + aff.shift).astype(np.float32)
    q, s = quantize_np(w.T.copy())
    p = ref.RefProgram(layers)
    wq, ws = p.op_weight(0)
    assert ws == s and np.array_equal(wq, q)
    assert p.labels() == ["NPU::FusedGemmAct(6->5, ReLU)"]
    x = rg.randn([3, 6])
    y = p.run(x)
    xq, xs = quantize_np(x)
    acc = xq.reshape(3, 6).astype(np.int64) @ q.reshape(5, 6).astype(np.int64).T
    val = ((acc.astype(np.float32) * np.float32(xs * s)).astype(np.float32) + b).astype(np.float32)
    assert_bitexact_f32(y, np.maximum(val, 0))


@pytest.mark.parametrize("c,o,k,s,p,h,w", [(3, 5, 3, 1, 1, 6, 7), (4, 6, 2, 2, 0, 7, 5), (2, 3, 3, 2, 2, 5, 5)])
def test_int8_conv_exact_per_image(ref, rg, c, o, k, s, p, h, w):
    """The INT8 conv of NpuProgram::execute (npu.rs:341-351) recomputed in
    numpy from brute-force im2col: per image, the transposed im2col matrix
    [L, C*k*k] (padding zeros included) is quantized with its own scale
    (quantize_into), multiplied exactly with the per-tensor weight
    quantization of [O, C*k*k], and the epilogue is act(fl(fl(acc) *
    fl(sa_b * sw)) + b).  The images differ in magnitude by up to 10^5, so
    one scale for the whole batch would change every other image's codes."""
    from rustgears_amd import nn
    rg.manual_seed(100 + c * 10 + k)
    conv = nn.Conv2d(c, o, k).stride(s).padding(p)
    layers = nn.Sequential().add(conv).add(nn.Relu()).export()
    n = 4
    x = rg.randn([n, c, h, w]) * np.array([1.0, 250.0, 0.003, 17.0], np.float32)[:, None, None, None]
    x = x.astype(np.float32)
    prog = ref.RefProgram(layers)
    prog.set_capture(True)
    y = prog.run(x)
    wq, sw = prog.op_weight(0)
    qw, sw_np = quantize_np(conv.weight.reshape(o, -1))
    assert sw == sw_np and np.array_equal(wq, qw)
    oh, ow = (h + 2 * p - k) // s + 1, (w + 2 * p - k) // s + 1
    L, ckk = oh * ow, c * k * k
    want_q, want_s, want_acc, want_y = [], [], [], []
    for b in range(n):
        cols_t = _im2col_brute(x[b], c, h, w, k, s, p).T.copy()  # [L, C*k*k]
        qa, sa = quantize_np(cols_t)
        acc = qa.reshape(L, ckk).astype(np.int64) @ qw.reshape(o, ckk).astype(np.int64).T  # [L, O]
        cs = np.float32(sa * sw)
        val = ((acc.astype(np.float32) * cs).astype(np.float32) + conv.bias).astype(np.float32)
        want_q.append(qa)
        want_s.append(sa)
        want_acc.append(acc.astype(np.int32))
        want_y.append(np.where(val > 0, val, np.float32(0)).T)  # NCHW: [O, L]
    assert np.array_equal(prog.capture(0, ref.CAP_QACT), np.concatenate(want_q))
    assert np.array_equal(prog.capture(0, ref.CAP_SCALE), np.array(want_s, np.float32))
    assert np.array_equal(prog.capture(0, ref.CAP_ACC), np.concatenate([a.reshape(-1) for a in want_acc]))
    assert_bitexact_f32(y, np.stack(want_y).reshape(n, o, oh, ow))
    # one scale per image: the scales differ, so a batch-wide scale would not match
    assert len(set(np.array(want_s).tolist())) == n


def test_lone_channel_affine_becomes_diagonal_gemm(ref):
    from rustgears_amd.inference import LayerSpec
    scale = np.array([2.0, -1.0, 0.5], np.float32)
    shift = np.array([0.1, 0.2, 0.3], np.float32)
    p = ref.RefProgram([LayerSpec.ChannelAffine(scale, shift)])
    assert p.labels() == ["NPU::Gemm(3->3)"]
    assert p.fp32_bytes == 0 and p.npu_bytes == 0  # no accounting (npu.rs:254-270)
    wq, ws = p.op_weight(0)
    assert wq.tolist() == [127, 0, 0, 0, -64, 0, 0, 0, 32] and ws == np.float32(np.float32(2.0) / np.float32(127))


def test_leaky_relu_label_rust_display(ref):
    from rustgears_amd.inference import Activation, LayerSpec
    for slope, txt in [(0.01, "0.01"), (0.2, "0.2"), (1.0, "1"), (1e-5, "0.00001"), (100.0, "100")]:
        layers = [LayerSpec.Linear(2, 2, np.ones(4, np.float32), np.zeros(2, np.float32)),
                  LayerSpec.Activation(Activation.leaky_relu(slope))]
        assert ref.RefProgram(layers).labels() == [f"NPU::FusedGemmAct(2->2, LeakyReLU({txt}))"]
        assert str(Activation.leaky_relu(slope)) == f"LeakyReLU({txt})"


def test_shape_errors(ref):
    from rustgears_amd.inference import LayerSpec
    p = ref.RefProgram([LayerSpec.Linear(3, 2, np.ones(6, np.float32), np.zeros(2, np.float32))])
    with pytest.raises(ValueError):
        p.run(np.ones((2, 4), np.float32))
    c = ref.RefProgram([LayerSpec.Conv2d(2, 1, 3, 1, 0, np.ones(18, np.float32), np.zeros(1, np.float32))])
    with pytest.raises(ValueError):
        c.run(np.ones((1, 3, 5, 5), np.float32))  # channel mismatch
    with pytest.raises(ValueError):
        c.run(np.ones((1, 2, 2, 2), np.float32))  # kernel larger than input


def test_golden_fixtures_reproduce(ref):
    """The committed fixtures (tests/golden/make_golden.py) still come out of
    the oracle bit for bit."""
    import golden_cases
    for case in golden_cases.load_all():
        p = ref.RefProgram(case["layers"])
        p.set_capture(True)
        y = p.run(case["x"])
        assert_bitexact_f32(y, case["y"], case["name"])
        for i, caps in enumerate(case["caps"]):
            for what, arr in caps.items():
                got = p.capture(i, what)
                if arr.dtype == np.float32:
                    assert_bitexact_f32(got, arr, f"{case['name']} op{i} cap{what}")
                else:
                    assert np.array_equal(got, arr), f"{case['name']} op{i} cap{what}"


# ---- NpuPrecision::Fp16 (npu.rs:425-445, quantize.rs:50-64) ---------------
def _bits(a):
    return np.asarray(a, np.float32).view(np.uint32)


def test_round_fp16_hand_vectors(ref):
    """Values derived by hand from quantize.rs:50-64: half an ulp added to the
    magnitude then truncated (ties away from zero), exponent < -14 -> +0
    (sign dropped), exponent > 15 -> +-65504 (NaN and inf included), and the
    exponent is taken before rounding, so 65520 becomes 65536."""
    cases = [(1.0, 1.0), (1 + 2**-11, 1 + 2**-10), (1 + 2**-11 - 2**-23, 1.0), (-(1 + 2**-11), -(1 + 2**-10)),
             (1 + 3 * 2**-11, 1 + 2**-9), (2**-14, 2**-14), (2**-15, 0.0), (-2**-15, 0.0), (1e-30, 0.0),
             (65504.0, 65504.0), (65519.9921875, 65504.0), (65520.0, 65536.0), (-65520.0, -65536.0),
             (65536.0, 65504.0), (1e9, 65504.0), (-np.inf, -65504.0), (np.inf, 65504.0), (np.nan, 65504.0),
             (0.1, 0.0999755859375), (-3.0, -3.0)]
    x = np.array([c[0] for c in cases], np.float32)
    want = np.array([c[1] for c in cases], np.float32)
    got = ref.round_fp16(x)
    assert np.array_equal(_bits(got), _bits(want)), list(zip(x, got, want))
    # -0 and tiny negatives flush to +0, not -0
    assert _bits(ref.round_fp16(np.float32(-0.0))) == 0 and _bits(ref.round_fp16(np.float32(-1e-30))) == 0


def test_round_fp16_vs_ieee_half_conversion(ref):
    """Against numpy's IEEE binary16 conversion (round to nearest even) over
    random normal-range values: equal except at exact ties, where
    round_fp16 always takes the larger magnitude."""
    rng = np.random.default_rng(5)
    e = rng.integers(-14, 16, 20000)
    x = (rng.uniform(1.0, 2.0, 20000) * np.exp2(e) * rng.choice([-1.0, 1.0], 20000)).astype(np.float32)
    # also exact ties: 12 significant bits with the last one set, normal range
    ties = ((2048 + 2 * rng.integers(0, 1024, 2000) + 1) / 4096.0 * np.exp2(rng.integers(-13, 16, 2000))).astype(np.float32)
    x = np.concatenate([x, ties, -ties])
    x = x[np.abs(x) < 65504]
    got = ref.round_fp16(x)
    ieee = x.astype(np.float16).astype(np.float32)
    tie = (_bits(x) & 0x1FFF) == 0x1000
    assert np.array_equal(_bits(got[~tie]), _bits(ieee[~tie]))
    up = np.sign(x[tie]) * (np.abs(x[tie]) + np.exp2(np.floor(np.log2(np.abs(x[tie]))) - 11))
    assert np.array_equal(_bits(got[tie]), _bits(up.astype(np.float32)))
    assert tie.sum() >= 3000


@pytest.mark.parametrize("m,k,n", [(3, 5, 4), (2, 17, 3), (1, 1, 1), (4, 33, 2)])
def test_fp16_gemm_serial_brute_force(ref, m, k, n):
    """fp16_gemm_fused against a scalar float32 loop in the reference's order:
    acc = 0; acc += round_fp16(a) * w (two roundings), then
    round_fp16(acc + bias) and ReLU."""
    rng = np.random.default_rng(m * 100 + k)
    a = (rng.standard_normal((m, k)) * 3).astype(np.float32)
    w = ref.round_fp16(rng.standard_normal((n, k)).astype(np.float32))
    b = rng.standard_normal(n).astype(np.float32)
    ah = ref.round_fp16(a)
    want = np.empty((m, n), np.float32)
    for r in range(m):
        for c in range(n):
            acc = np.float32(0.0)
            for j in range(k):
                acc = np.float32(acc + np.float32(ah[r, j] * w[c, j]))
            want[r, c] = max(np.float32(ref.round_fp16(np.float32(acc + b[c])).item()), np.float32(0.0))
    assert_bitexact_f32(ref.fp16_gemm_fused(a, w, b, act=1), want)


def test_fp16_program_linear_and_accounting(ref, rg):
    """FP16 programs: weights rounded with round_fp16 after the transpose,
    npu bytes = 2 per weight and bias element (npu.rs:210-215), and the run is
    the chain of fp16_gemm_fused calls."""
    from rustgears_amd import nn
    rg.manual_seed(31)
    l1, l2 = nn.Linear(7, 9), nn.Linear(9, 4)
    layers = nn.Sequential().add(l1).add(nn.Relu()).add(l2).export()
    p = ref.RefProgram(layers, precision=ref.FP16)
    assert p.labels() == ["NPU::FusedGemmAct(7->9, ReLU)", "NPU::Gemm(9->4)"]
    assert p.npu_bytes == (7 * 9 + 9 + 9 * 4 + 4) * 2 and p.fp32_bytes == (7 * 9 + 9 + 9 * 4 + 4) * 4
    x = rg.randn([5, 7])
    h = ref.fp16_gemm_fused(x, ref.round_fp16(l1.weight.T.copy()), l1.bias, act=1)
    y = ref.fp16_gemm_fused(h, ref.round_fp16(l2.weight.T.copy()), l2.bias)
    assert_bitexact_f32(p.run(x), y)


def test_fp16_lone_channel_affine_is_elementwise(ref):
    """A lone ChannelAffine in FP16 multiplies by the raw (unrounded) scale
    (npu.rs:254-270): the serial sum has one non-zero term, so
    y = round_fp16(fl(round_fp16(x) * scale) + shift)."""
    from rustgears_amd.inference import LayerSpec
    rng = np.random.default_rng(9)
    scale = rng.standard_normal(6).astype(np.float32) * np.float32(1.0001)
    shift = rng.standard_normal(6).astype(np.float32)
    p = ref.RefProgram([LayerSpec.ChannelAffine(scale, shift)], precision=ref.FP16)
    x = (rng.standard_normal((4, 6)) * 7).astype(np.float32)
    want = ref.round_fp16((ref.round_fp16(x) * scale).astype(np.float32) + shift)
    assert_bitexact_f32(p.run(x), want)


def test_fp16_conv_is_im2col_gemm(ref):
    """FP16 Conv2d per image: im2col, transpose, fp16_gemm_fused with the
    rounded [out, c*k*k] weights, transpose back (npu.rs:341-376)."""
    from rustgears_amd.inference import LayerSpec
    rng = np.random.default_rng(4)
    c, o, k, h, w = 3, 5, 3, 7, 6
    wt = rng.standard_normal((o, c, k, k)).astype(np.float32)
    b = rng.standard_normal(o).astype(np.float32)
    p = ref.RefProgram([LayerSpec.Conv2d(c, o, k, 1, 1, wt.ravel(), b)], precision=ref.FP16)
    x = rng.standard_normal((2, c, h, w)).astype(np.float32)
    y = p.run(x)
    for i in range(2):
        cols = _im2col_brute(x[i], c, h, w, k, 1, 1)  # [ckk, L]
        ylo = ref.fp16_gemm_fused(cols.T.copy(), ref.round_fp16(wt.reshape(o, -1)), b)
        assert_bitexact_f32(y[i], ylo.T.reshape(o, h, w))


# ---- standard FP32 path (run_standard, mod.rs:260-331) ----------------------
@pytest.mark.parametrize("m,k,n", [(3, 5, 4), (2, 17, 3), (1, 1, 1)])
def test_standard_matmul_serial_order(ref, m, k, n):
    """rgref_matmul_f32: per output a serial float32 sum over k in order,
    multiply then add (the WGSL shader's order, wgpu_impl.rs:20-48)."""
    rng = np.random.default_rng(m + 10 * k)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c = np.empty((m, n), np.float32)
    ref.lib().rgref_matmul_f32(ref._fp(a), ref._fp(b), m, k, n, ref._fp(c), 0)
    want = np.empty((m, n), np.float32)
    for r in range(m):
        for j in range(n):
            acc = np.float32(0.0)
            for p in range(k):
                acc = np.float32(acc + np.float32(a[r, p] * b[p, j]))
            want[r, j] = acc
    assert_bitexact_f32(c, want)


@pytest.mark.parametrize("m,k,n,par", [(2, 9, 600, 0), (1, 40, 257, 1), (5, 33, 513, 1), (64, 3, 1, 1)])
def test_standard_matmul_column_blocks(ref, m, k, n, par):
    """The same serial order across several (and ragged) column blocks, with
    and without the parallel split: numpy's elementwise float32 products and
    sums, accumulated over k in order."""
    rng = np.random.default_rng(m * 7 + n)
    a = rng.standard_normal((m, k)).astype(np.float32)
    b = rng.standard_normal((k, n)).astype(np.float32)
    c = np.empty((m, n), np.float32)
    ref.lib().rgref_matmul_f32(ref._fp(a), ref._fp(b), m, k, n, ref._fp(c), par)
    acc = np.zeros((m, n), np.float32)
    for p in range(k):
        acc = acc + (a[:, p:p + 1] * b[p:p + 1, :])
    assert acc.dtype == np.float32
    assert_bitexact_f32(c, acc)


def test_standard_program_linear_bn_relu(ref, rg):
    """Standard program: BN folded like the NPU compile (mod.rs:168-171), then
    matmul with the exported [in, out] weights, the bias added separately,
    and ReLU as its own layer."""
    from rustgears_amd import nn
    rg.manual_seed(77)
    lin, bn = nn.Linear(6, 5), nn.BatchNorm1d(5)
    bn.running_mean = rg.randn([5])
    bn.running_var = rg.uniform([5], 0.5, 1.5)
    layers = nn.Sequential().add(lin).add(bn).add(nn.Relu()).export()
    aff = layers[1]
    w = (lin.weight * aff.scale[None, :]).astype(np.float32)
    b = ((lin.bias * aff.scale).astype(np.float32) + aff.shift).astype(np.float32)
    x = rg.randn([3, 6])
    mm = np.empty((3, 5), np.float32)
    ref.lib().rgref_matmul_f32(ref._fp(np.ascontiguousarray(x)), ref._fp(np.ascontiguousarray(w)), 3, 6, 5,
                               ref._fp(mm), 0)
    p = ref.RefProgram(layers, precision=ref.FP32)
    assert p.num_ops == 2  # Linear (BN folded) and Activation
    assert_bitexact_f32(p.run(x), np.maximum((mm + b).astype(np.float32), 0))


def test_standard_program_affine_and_conv(ref):
    """A ChannelAffine that does not fold is v * scale + shift per channel on
    axis 1 (mod.rs:292-306); conv is im2col then W[O, ckk] @ cols plus the
    bias per channel (kernels.rs:218-265)."""
    from rustgears_amd.inference import LayerSpec
    rng = np.random.default_rng(2)
    sc = rng.standard_normal(3).astype(np.float32)
    sh = rng.standard_normal(3).astype(np.float32)
    x = rng.standard_normal((2, 3, 4, 5)).astype(np.float32)
    p = ref.RefProgram([LayerSpec.ChannelAffine(sc, sh)], precision=ref.FP32)
    assert_bitexact_f32(p.run(x), (x * sc[None, :, None, None]).astype(np.float32) + sh[None, :, None, None])
    w = rng.standard_normal((4, 3, 3, 3)).astype(np.float32)
    bias = rng.standard_normal(4).astype(np.float32)
    p = ref.RefProgram([LayerSpec.Conv2d(3, 4, 3, 1, 1, w.ravel(), bias)], precision=ref.FP32)
    y = p.run(x)
    for i in range(2):
        cols = np.ascontiguousarray(_im2col_brute(x[i], 3, 4, 5, 3, 1, 1))
        mm = np.empty((4, 20), np.float32)
        ref.lib().rgref_matmul_f32(ref._fp(np.ascontiguousarray(w.reshape(4, -1))), ref._fp(cols), 4, 27, 20,
                                   ref._fp(mm), 0)
        assert_bitexact_f32(y[i], (mm + bias[:, None]).astype(np.float32).reshape(4, 4, 5))
