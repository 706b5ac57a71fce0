"""ExecutionProvider::Gpu(i): the standard FP32 path (run_standard,
mod.rs:260-331) on the MI355X against the CPU oracle's restatement.

The reference's matmul order depends on its backend (the WGSL shader sums
serially in k, the CPU backend blocks with FMA), so no single bit pattern is
the reference's; the oracle sums serially in k.  Any f32 summation of K
products is within K u sum|p| of the exact sum (u = 2^-24, products
included), so the GPU's f32 MFMA sums and the oracle's are within
B = (2K + 4) u (sum|p| + |b|) + 2 u |y| of each other after the bias add.
Each op is checked on the GPU's own captured input; the elementwise layers
(ChannelAffine, activations, pool, softmax) must match bit for bit.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu

CAP_OUT = 3
U = 2.0 ** -24


def make_session(rg, layers, device=0):
    return rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.Gpu(device))


def folded_groups(layers):
    """Raw layers grouped as the folded program's ops: a Linear/Conv2d with
    the ChannelAffine layers that fold into it (fold_batch_norm, mod.rs:225-257),
    every other layer alone."""
    from rustgears_amd.inference import LayerSpec
    groups, i = [], 0
    while i < len(layers):
        g = [layers[i]]
        i += 1
        if isinstance(g[0], (LayerSpec.Linear, LayerSpec.Conv2d)):
            out = g[0].out_features if isinstance(g[0], LayerSpec.Linear) else g[0].out_channels
            while i < len(layers) and isinstance(layers[i], LayerSpec.ChannelAffine) and len(layers[i].scale) == out:
                g.append(layers[i])
                i += 1
        groups.append(g)
    return groups


def check_bound(got, want, a, w_kn, bias, what):
    """got/want [m, n]; a [m, k]; w_kn [k, n] (folded weights)."""
    k = a.shape[1]
    sum_abs = np.abs(a.astype(np.float64)) @ np.abs(w_kn.astype(np.float64))
    bound = (2 * k + 4) * U * (sum_abs + np.abs(bias.astype(np.float64))[None, :]) + 2 * U * np.abs(want) + 1e-38
    diff = np.abs(got.astype(np.float64) - want.astype(np.float64))
    bad = np.flatnonzero(~(diff <= bound))
    assert bad.size == 0, (f"{what}: {bad.size} outside the bound, first {bad[:5]} got {got.ravel()[bad[:5]]} "
                           f"want {want.ravel()[bad[:5]]}")
    exact = np.mean(got.view(np.uint32) == want.view(np.uint32))
    print(f"[fp32] {what}: max |diff| {diff.max():.3g}, bit-equal {exact:.4f}", flush=True)


def folded_weight(ref, group):
    """The folded [k, n] weights and bias of a Linear/Conv group, folded in
    numpy as fold_batch_norm does (f32: w *= scale, b = b * scale + shift);
    used only for the error bound."""
    from rustgears_amd.inference import LayerSpec
    head = group[0]
    if isinstance(head, LayerSpec.Linear):
        w = head.weight.reshape(head.in_features, head.out_features).copy()
        b = head.bias.copy()
        for aff in group[1:]:
            w = (w * aff.scale[None, :]).astype(np.float32)
            b = ((b * aff.scale).astype(np.float32) + aff.shift).astype(np.float32)
        return w, b
    o = head.out_channels
    w = head.weight.reshape(o, -1).copy()
    b = head.bias.copy()
    for aff in group[1:]:
        w = (w * aff.scale[:, None]).astype(np.float32)
        b = ((b * aff.scale).astype(np.float32) + aff.shift).astype(np.float32)
    return w.T.copy(), b  # [ckk, O]


def check_per_op(rg, ref, layers, x, what):
    from rustgears_amd.inference import LayerSpec
    print(f"[fp32] {what} x{tuple(x.shape)}", flush=True)
    sess = make_session(rg, layers)
    sess.set_capture(True)
    y = sess.run(x)
    groups = folded_groups(layers)
    p_all = ref.RefProgram(layers, precision=ref.FP32)
    assert p_all.num_ops == len(groups) == len(sess.op_labels()), what
    inp = x
    for i, g in enumerate(groups):
        p = ref.RefProgram(g, precision=ref.FP32)
        want = p.run(inp)
        got = sess.capture(i, CAP_OUT)
        assert got.size == want.size, f"{what} op{i}"
        got = got.reshape(want.shape)
        head = g[0]
        if isinstance(head, LayerSpec.Linear):
            w, b = folded_weight(ref, g)
            a = inp.reshape(-1, head.in_features)
            check_bound(got.reshape(a.shape[0], -1), want.reshape(a.shape[0], -1), a, w, b, f"{what} op{i}")
        elif isinstance(head, LayerSpec.Conv2d):
            w, b = folded_weight(ref, g)
            n, c = inp.shape[0], inp.shape[1]
            k, s, pd, o = head.kernel, head.stride, head.padding, head.out_channels
            oh, ow = got.shape[2], got.shape[3]
            xp = np.pad(inp, ((0, 0), (0, 0), (pd, pd), (pd, pd)))
            cols = np.empty((n, oh * ow, c * k * k), np.float32)
            for ci in range(c):
                for ki in range(k):
                    for kj in range(k):
                        cols[:, :, (ci * k + ki) * k + kj] = xp[:, ci, ki:ki + s * oh:s, kj:kj + s * ow:s].reshape(n, -1)
            g2 = np.ascontiguousarray(got.transpose(0, 2, 3, 1).reshape(-1, o))
            w2 = np.ascontiguousarray(want.transpose(0, 2, 3, 1).reshape(-1, o))
            check_bound(g2, w2, cols.reshape(-1, c * k * k), w, b, f"{what} op{i}")
        else:
            assert_bitexact_f32(got, want, f"{what} op{i}")
        inp = got
    assert sess.last_npu_profile() is None
    sess.close()
    return y


def test_fp32_deep_mlp_per_op(rg, ref):
    from rustgears_amd import configs
    model, x = configs.deep_mlp(rows=300)
    check_per_op(rg, ref, model.export(), x, "deep_mlp fp32")


@pytest.mark.parametrize("rows", [1, 5, 8, 255, 700, 4200])
def test_fp32_rows_gemv_and_gemm(rg, ref, rows):
    from rustgears_amd import nn
    rg.manual_seed(rows + 3)
    m = nn.Sequential().add(nn.Linear(300, 400)).add(nn.Gelu()).add(nn.Linear(400, 9))
    check_per_op(rg, ref, m.export(), rg.randn([rows, 300]), f"rows {rows}")


def test_fp32_cnn_per_op(rg, ref):
    from rustgears_amd import configs
    model, x = configs.cnn(n=8)
    check_per_op(rg, ref, model.export(), x, "cnn fp32")


def test_fp32_lone_affine_and_standalone_ops(rg, ref):
    """A ChannelAffine that cannot fold stays elementwise (not the NPU's
    diagonal Linear), on NCHW and on rows."""
    from rustgears_amd.inference import Activation, LayerSpec
    rg.manual_seed(12)
    layers = [LayerSpec.MaxPool2d(2, 2), LayerSpec.ChannelAffine(rg.randn([3]), rg.randn([3])),
              LayerSpec.Activation(Activation.TANH), LayerSpec.Flatten(),
              LayerSpec.Linear(3 * 4 * 4, 6, rg.randn([48 * 6]), rg.randn([6])), LayerSpec.Softmax()]
    check_per_op(rg, ref, layers, rg.randn([4, 3, 8, 8]), "pool/affine/tanh/flatten/linear/softmax")
    rows = [LayerSpec.ChannelAffine(rg.randn([7]), rg.randn([7])), LayerSpec.Activation(Activation.leaky_relu(0.1))]
    check_per_op(rg, ref, rows, rg.randn([5, 7]), "affine rows")


def test_fp32_report(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(0)
    model = nn.Sequential().add(nn.Linear(16, 64)).add(nn.BatchNorm1d(64)).add(nn.Relu()).add(nn.Linear(64, 4))
    sess = make_session(rg, model.export())
    # compilation_report of a Standard program (mod.rs:198-204): 3 folded layers from 4 raw ones
    assert sess.compilation_report() == "InferenceSession [provider = GPU:0 (FP32), device = gpu:0, ops = 3 (from 4 raw layers)]"
    sess.close()


@pytest.mark.parametrize("spec", [(3, 32, 3, 1, 1), (2, 5, 3, 2, 0), (1, 64, 5, 1, 2), (7, 4, 2, 1, 0), (3, 17, 3, 3, 1)])
def test_fp32_direct_conv_exact(rg, ref, spec):
    """A convolution whose window holds at most 32 values runs as a direct
    conv that sums the taps in the reference's serial im2col order, so it is
    bit-exact with the oracle (not only within the reordering bound)."""
    from rustgears_amd import nn
    C, O, k, s, p = spec
    rg.manual_seed(C * 100 + O * 10 + k)
    m = nn.Sequential().add(nn.Conv2d(C, O, k).stride(s).padding(p)).add(nn.Relu())
    layers = m.export()
    x = (rg.randn([4, C, 11, 13]) * 2.0).astype(np.float32)
    print(f"[direct conv fp32] {spec}", flush=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.Gpu(0))
    y = sess.run(x)
    want = ref.RefProgram(layers, precision=ref.FP32).run(x)
    assert_bitexact_f32(y, want, f"direct conv {spec}")
    sess.close()


@pytest.mark.parametrize("seed", range(32))
def test_fp32_random_models(rg, ref, seed):
    """The INT8 suite's seeded random layer stacks on this provider: every
    Linear/Conv op within the summation-order bound, every other op bit for
    bit."""
    from test_gpu_parity import _random_model
    layers, x = _random_model(1000 + seed)
    check_per_op(rg, ref, layers, x, f"random model {seed}")
