"""The next Linear's quantization fused into the producing GEMM (requant.hip).

An INT8 Linear whose next computing op is a Linear quantizes that op's input
itself: a persistent grid computes its tiles, meets at a grid barrier on the
per-tensor absmax (npu.rs:312, quantize.rs:18-24), and quantizes its own
tiles -- the last one from registers, earlier ones from their stored f32
outputs.  These tests check, bit for bit against the oracle:

* runs without capture (the last tiles' f32 outputs are never written) and
  with capture (every tap: i8 operand, scale, i32 sums, f32 outputs);
* workgroups that walk several tiles (more 256 x 256 tiles than CUs), every
  tile shape, ragged M and N (padding columns within a tile; an N that is not
  a multiple of 4 keeps the separate quantize pass), activations whose value
  at 0 is not 0 (the padding columns must not reach the absmax), and chains
  of three and four fused Linears (the two i8 operand buffers alternate);
* the deferral path: with RGNPU_REQUANT_SPIN_LIMIT=0 no workgroup waits at
  the barrier, and the finisher quantizes every other workgroup's tiles;
* that a fused consumer launches nothing before its GEMM (its op time equals
  its kernel time in the profile);
* the one-pass quantization of a Linear's own input (a persistent grid that
  keeps its share of the input in registers and LDS across the barrier): an
  input larger than what the grid keeps (the rest is read twice), with and
  without deferral.
"""
import numpy as np
import pytest

from conftest import assert_bitexact_f32
from test_gpu_parity import check_against_oracle

pytestmark = pytest.mark.gpu


def _chain(rg, dims, act, seed):
    from rustgears_amd import nn
    rg.manual_seed(seed)
    m = nn.Sequential()
    for a, b in zip(dims[:-1], dims[1:]):
        m.add(nn.Linear(a, b))
        if act is not None:
            m.add(act())
    return m.export()


def _rup(v, m):
    return (v + m - 1) // m * m


def _unsplit(mpad, npad, kpad):
    """The large GEMM's choice (kernels.hip choose_gemm): False when K is split."""
    if mpad % 256 == 0 and npad % 256 == 0 and (mpad // 256) * (npad // 256) >= 256:
        return True
    if mpad % 256 == 0 and npad % 128 == 0 and (mpad // 256) * (npad // 128) >= 256:
        return True
    tiles, nk = (mpad // 128) * (npad // 128), kpad // 64
    if tiles >= 128:
        return True
    s = max(1, min(512 // max(tiles, 1), nk // 4))
    ks = -(-nk // s)
    return -(-nk // ks) == 1


def _expected_fused(dims, rows):
    """Per Linear after the first: is its input quantized by its producer?
    (producer on the unsplit MFMA GEMM -- more than 8 rows, more than 16
    outputs -- with a multiple of 4 outputs)"""
    mpad = _rup(rows, 256)
    out = []
    for k, n, n2 in zip(dims[:-2], dims[1:-1], dims[2:]):
        out.append(rows > 8 and n > 16 and n % 4 == 0 and _unsplit(mpad, _rup(n, 256), _rup(k, 128)))
    return out


def _expected_small_xq(dims, rows, fused):
    """Per Linear after the first: does it quantize its input as it reads it
    in the small-tile GEMM (program.cpp make_plan small_xq)?  Not fused, more
    than 8 rows and 16 outputs, not itself a fused producer, fewer than 128
    tiles of 128 x 128, K % 4 == 0, at most 512 blocks of 16 rows."""
    mpad = _rup(rows, 256)
    out = []
    for c in range(1, len(dims) - 1):
        k, n = dims[c], dims[c + 1]
        npad = _rup(n, 256)
        producer = c < len(dims) - 2 and fused[c]
        blocks = -(-rows // 16) * (npad // 64)
        out.append(not fused[c - 1] and rows > 8 and n > 16 and not producer and
                   (mpad // 128) * (npad // 128) < 128 and k % 4 == 0 and blocks <= 512)
    return out


def _run_plain(rg, ref, layers, x, what):
    print(f"[requant] {what} x{tuple(x.shape)}", flush=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    y2 = sess.run(x)  # a second run on the same plan (slot sets alternate)
    prof = sess.last_npu_profile()
    sess.close()
    want = ref.RefProgram(layers).run(x, parallel=True)
    assert_bitexact_f32(y, want, what)
    assert_bitexact_f32(y2, want, what + " (second run)")
    return prof


CASES = [
    # (name, dims, act, rows): tile shape in the comment (256x256 with > 256
    # tiles means several tiles per workgroup)
    ("multi-tile 256x256 gelu", [4000, 4000, 4000], "gelu", 4400),      # 18 x 16 = 288 tiles
    ("256x128 relu", [1000, 3000, 2000, 500], "relu", 2600),             # 11 x 24 tiles
    ("128x128 sigmoid ragged n", [700, 2004, 1516, 300], "sigmoid", 1500),  # 1516 -> 300 splits K
    ("ragged n leaky", [333, 260, 259, 20], "leaky", 777),  # 259 % 4 != 0: not fused
    ("four fused tanh", [256, 384, 512, 384, 130], "tanh", 300),
]


def _act(nn, name):
    return {"gelu": nn.Gelu, "relu": nn.Relu, "sigmoid": nn.Sigmoid, "tanh": nn.Tanh,
            "leaky": lambda: nn.LeakyRelu(0.03), None: None}[name]


@pytest.mark.parametrize("name,dims,act,rows", CASES, ids=[c[0] for c in CASES])
def test_fused_requant_without_capture(rg, ref, name, dims, act, rows):
    from rustgears_amd import nn
    layers = _chain(rg, dims, _act(nn, act), seed=rows + len(dims))
    x = rg.randn([rows, dims[0]])
    prof = _run_plain(rg, ref, layers, x, name)
    gemm_ops = [r for r in prof.records if "Gemm" in r.op]
    fused = _expected_fused(dims, rows)
    assert any(fused), "the case must exercise the fused path"
    # a Linear whose operand its producer quantized, or that quantizes its
    # input as it reads it, launches nothing before its GEMM; the others run
    # their absmax / quantize kernels first
    for r, f, sx in zip(gemm_ops[1:], fused, _expected_small_xq(dims, rows, fused)):
        assert (r.duration_ns == r.kernel_ns) == (f or sx), (r, f, sx)


@pytest.mark.parametrize("name,dims,act,rows", CASES[:3] + CASES[4:], ids=[c[0] for c in CASES[:3] + CASES[4:]])
def test_fused_requant_capture_taps(rg, ref, name, dims, act, rows):
    from rustgears_amd import nn
    layers = _chain(rg, dims, _act(nn, act), seed=rows + len(dims))
    check_against_oracle(rg, ref, layers, rg.randn([rows, dims[0]]), name)


@pytest.mark.parametrize("name,dims,act,rows", [CASES[0], CASES[2], CASES[4]], ids=[CASES[0][0], CASES[2][0],
                                                                                   CASES[4][0]])
def test_deferred_quantization_by_the_finisher(rg, ref, monkeypatch, name, dims, act, rows):
    """No workgroup waits at the barrier: each one that is not last stores its
    outputs and defers, and the finisher quantizes all of their tiles."""
    from rustgears_amd import nn
    monkeypatch.setenv("RGNPU_REQUANT_SPIN_LIMIT", "0")
    layers = _chain(rg, dims, _act(nn, act), seed=rows + len(dims))
    x = rg.randn([rows, dims[0]])
    _run_plain(rg, ref, layers, x, name + " (deferred)")
    check_against_oracle(rg, ref, layers, x, name + " (deferred, capture)")


def test_linear_stack_full_without_capture(rg, ref):
    """The benchmark config (4 x 4096^2 GELU, 8192 rows) on the fused path,
    without capture taps, against the oracle's output."""
    from rustgears_amd import configs
    model, x = configs.linear_stack()
    layers = model.export()
    prof = _run_plain(rg, ref, layers, x, "stack 4096 gelu full (no capture)")
    assert _expected_fused([4096] * 5, 8192) == [True] * 3
    for r in prof.records[1:]:
        assert r.duration_ns == r.kernel_ns, r


@pytest.mark.parametrize("spin", [None, "0"], ids=["resident", "deferred"])
def test_input_quantization_larger_than_the_grid_keeps(rg, ref, monkeypatch, spin):
    """8192 x 8192 f32 (256 MiB) into Linear(8192, 40): 32 chunks of 16
    inputs per thread of a 256-workgroup grid, 16 of them kept; the i8
    operand and scale taps are compared with the oracle's."""
    from rustgears_amd import nn
    if spin is not None:
        monkeypatch.setenv("RGNPU_REQUANT_SPIN_LIMIT", spin)
    rg.manual_seed(41)
    layers = nn.Sequential().add(nn.Linear(8192, 40)).add(nn.Relu()).export()
    x = rg.randn([8192, 8192])
    x[5, 7] = -93.25  # the absmax sits in the first kept chunk of one thread
    check_against_oracle(rg, ref, layers, x, f"input quant 8192x8192 spin={spin}")
