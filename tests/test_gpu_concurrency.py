"""Concurrent InferenceSession.run on one session (run(&self) is Sync,
mod.rs:146-151, 212-221): host-pointer runs from several threads borrow
separate workers (own stream, plans, absmax slots) that share the device
weights.  Every concurrent result must equal the serial one bit for bit,
whatever the interleaving, and the profile stays a complete profile."""
from concurrent.futures import ThreadPoolExecutor

import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("prec", ["int8", "fp16", "fp32"])
def test_concurrent_runs_match_serial(rg, ref, prec):
    from rustgears_amd import configs
    model, _ = configs.deep_mlp(rows=384)
    provider = {"int8": rg.ExecutionProvider.mi355x_int8(), "fp16": rg.ExecutionProvider.mi355x_fp16(),
                "fp32": rg.ExecutionProvider.Gpu(0)}[prec]
    layers = model.export()
    sess = rg.InferenceSession.from_layers(layers, provider)
    # different magnitudes and row counts: a shared slot or buffer between
    # concurrent runs would change scales or shapes
    inputs = [(rg.randn([384 if i % 3 else 200, 784]) * (0.1 + i)).astype(np.float32) for i in range(8)]
    want = [sess.run(x) for x in inputs]
    print(f"[concurrency] {prec}: 6 threads x {3 * len(inputs)} runs", flush=True)
    with ThreadPoolExecutor(6) as ex:
        got = list(ex.map(sess.run, inputs * 3))
    for i, (g, w) in enumerate(zip(got, want * 3)):
        assert_bitexact_f32(g, w, f"{prec} run {i}")
    if prec == "int8":
        assert_bitexact_f32(want[0], ref.RefProgram(layers).run(inputs[0]), "int8 vs oracle")
        prof = sess.last_npu_profile()
        assert prof is not None and prof.fused_ops == 3 and len(prof.records) == 3
    sess.close()


def test_concurrent_runs_with_device_runs_and_capture(rg, ref):
    """Host runs on workers while the handle's own stream serves
    run_device; capture mode runs on the handle and stays exact."""
    from rustgears_amd import configs
    model, x = configs.deep_mlp(rows=256)
    layers = model.export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    want = sess.run(x)
    dx = rg.DeviceBuffer.from_array(x)
    dy = rg.DeviceBuffer(want.nbytes)
    with ThreadPoolExecutor(4) as ex:
        futs = [ex.submit(sess.run, x) for _ in range(8)]
        for _ in range(4):
            sess.run_device(dx, x.shape, dy)
        sess.synchronize()
        for f in futs:
            assert_bitexact_f32(f.result(), want, "host run beside run_device")
    assert_bitexact_f32(dy.download(want.shape), want, "run_device")
    sess.set_capture(True)
    y = sess.run(x)
    assert_bitexact_f32(y, want, "capture run")
    assert_bitexact_f32(sess.capture(2, 3).reshape(want.shape), want, "capture tap")
    sess.close()


@pytest.mark.parametrize("rows", [255, 256, 1023, 2049, 10000])
def test_staged_host_copies(rg, ref, rows):
    """run() moves inputs and outputs of 1 MiB and more through the pinned
    staging ring, in chunks of a quarter of the copy between 1 and 8 MiB:
    255 rows x 1024 f32 stays below 1 MiB (plain copy), 256 rows is one
    1 MiB chunk, 1023 and 2049 rows end in a ragged chunk, and 10000 rows
    (8 MiB chunks) needs more chunks than the ring's 4 slots.  The result
    equals the device-resident run bit for bit."""
    from rustgears_amd import configs
    model, _ = configs.linear_stack(rows=rows, width=1024, depth=2)
    layers = model.export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    x = (rg.randn([rows, 1024]) * 3.0).astype(np.float32)
    print(f"[staging] rows={rows} in={x.nbytes} bytes", flush=True)
    y = sess.run(x)
    dx = rg.DeviceBuffer.from_array(x)
    dy = rg.DeviceBuffer(y.nbytes)
    sess.run_device(dx, x.shape, dy)
    sess.synchronize()
    assert_bitexact_f32(y, dy.download(y.shape), f"host vs device run, rows {rows}")
    assert_bitexact_f32(sess.run(x), y, "second host run")
    if rows == 2049:
        assert_bitexact_f32(y, ref.RefProgram(layers).run(x), "staged run vs oracle")
    sess.close()


def test_staged_input_small_output_and_concurrency(rg):
    """A staged input with an output below the staging size, then several
    threads each moving ~40 MB each way on their own worker ring."""
    from rustgears_amd import configs
    model, _ = configs.deep_mlp(rows=6000, d_in=1024, hidden=1024, d_out=10)
    sess = rg.InferenceSession.from_layers(model.export(), rg.ExecutionProvider.mi355x_int8())
    x = rg.uniform([6000, 1024], 0.0, 1.0).astype(np.float32)
    y = sess.run(x)
    dx = rg.DeviceBuffer.from_array(x)
    dy = rg.DeviceBuffer(y.nbytes)
    sess.run_device(dx, x.shape, dy)
    sess.synchronize()
    assert_bitexact_f32(y, dy.download(y.shape), "staged input, small output")
    sess.close()

    model, _ = configs.linear_stack(rows=10000, width=1024, depth=1)
    sess = rg.InferenceSession.from_layers(model.export(), rg.ExecutionProvider.mi355x_int8())
    xs = [(rg.randn([10000, 1024]) * (1 + i)).astype(np.float32) for i in range(4)]
    want = [sess.run(x) for x in xs]
    print("[staging] 4 threads x 12 runs of 41 MB", flush=True)
    with ThreadPoolExecutor(4) as ex:
        got = list(ex.map(sess.run, xs * 3))
    for i, (g, w) in enumerate(zip(got, want * 3)):
        assert_bitexact_f32(g, w, f"concurrent staged run {i}")
    sess.close()


@pytest.mark.parametrize("name", ["cnn", "quickstart"])
def test_concurrent_runs_of_one_kernel_programs(rg, ref, name):
    """Six threads on the CNN (both convs and pools in one workgroup per
    image, the fc layer adding its K slices through counting atomics in the
    run's slot set, the head quantizing its input as it reads it) and on the
    quickstart MLP (the whole program in one workgroup): two batch sizes and
    input magnitudes interleaved, every result bit-exact with the serial run
    of the same input and the serial runs with the oracle."""
    from rustgears_amd import configs
    if name == "cnn":
        model, x0 = configs.cnn(n=256)
        sizes = [256, 96]
    else:
        model, x0 = configs.quickstart(rows=64)
        sizes = [64, 17]
    layers = model.export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    inputs = [(rg.randn([sizes[i % 2]] + list(x0.shape[1:])) * (0.1 + i)).astype(np.float32) for i in range(6)]
    want = [sess.run(x) for x in inputs]
    print(f"[concurrency] {name}: 6 threads x {3 * len(inputs)} runs", flush=True)
    with ThreadPoolExecutor(6) as ex:
        got = list(ex.map(sess.run, inputs * 3))
    for i, (g, w) in enumerate(zip(got, want * 3)):
        assert_bitexact_f32(g, w, f"{name} run {i}")
    for i in range(2):
        assert_bitexact_f32(want[i], ref.RefProgram(layers).run(inputs[i], parallel=True), f"{name} {i} vs oracle")
    sess.close()
