"""NpuProfile bookkeeping on the device (npu.rs:296-421, mod.rs:193-195, 217).

* A device run's profile stays readable after a shape-only query replaced the
  handle's plan, and a completed host run supersedes a device run whose
  profile was never read.
* Every op of a run is timed, also when its convs launch four kernels each
  (FP16 im2col + GEMM + split-K epilogue + NCHW transpose).
* The first run of a fresh process reports microsecond-scale op times: the
  code object is loaded when the program is created, not inside the run.
"""
import ctypes
import os
import subprocess
import sys

import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _mlp(rg):
    from rustgears_amd import nn
    rg.manual_seed(19)
    return nn.Sequential().add(nn.Linear(16, 32)).add(nn.Relu()).add(nn.Linear(32, 4)).export()


def test_device_run_profile_survives_shape_query(rg, ref):
    from rustgears_amd import _native as N
    from rustgears_amd.inference import DeviceBuffer
    layers = _mlp(rg)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    x = rg.randn([64, 16])
    d_x, d_y = DeviceBuffer.from_array(x), DeviceBuffer(64 * 4 * 4)
    assert sess.run_device(d_x, x.shape, d_y) == (64, 4)
    # shape-only query on the handle itself: a new plan for 300 rows
    sh = (ctypes.c_int64 * 2)(300, 16)
    shp = (ctypes.c_int64 * 8)()
    nd = ctypes.c_int32()
    N.check(N.lib().rgnpu_program_run_device(sess._h, None, sh, 2, None, 0, shp, ctypes.byref(nd)))
    assert tuple(shp[i] for i in range(nd.value)) == (300, 4)
    prof = sess.last_npu_profile()
    assert [r.macs for r in prof.records] == [64 * 16 * 32, 64 * 32 * 4]
    # the two Linears run as one kernel (mlp_tiny_kernel): the first op's
    # record holds its time and the second op launches nothing
    assert prof.records[0].duration_ns > 0 and prof.records[1].duration_ns == 0, prof.records
    assert_bitexact_f32(d_y.download((64, 4)), ref.RefProgram(layers).run(x), "device run")
    sess.close()


def test_host_run_supersedes_pending_device_run(rg, ref):
    from rustgears_amd.inference import DeviceBuffer
    layers = _mlp(rg)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    x = rg.randn([64, 16])
    d_x, d_y = DeviceBuffer.from_array(x), DeviceBuffer(64 * 4 * 4)
    sess.run_device(d_x, x.shape, d_y)
    x2 = rg.randn([10, 16])
    y2 = sess.run(x2)
    prof = sess.last_npu_profile()
    assert [r.macs for r in prof.records] == [10 * 16 * 32, 10 * 32 * 4]
    assert_bitexact_f32(y2, ref.RefProgram(layers).run(x2), "host run")
    sess.synchronize()
    # the device run's profile never replaces the newer one
    assert [r.macs for r in sess.last_npu_profile().records] == [10 * 16 * 32, 10 * 32 * 4]
    sess.close()


def test_every_op_timed_with_four_launch_convs(rg, ref):
    from rustgears_amd import nn
    rg.manual_seed(23)
    m = nn.Sequential()
    for _ in range(4):
        m.add(nn.Conv2d(64, 64, 3).padding(1)).add(nn.Relu())
    m.add(nn.MaxPool2d(2)).add(nn.Flatten()).add(nn.Linear(64 * 4 * 4, 10))
    layers = m.export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_fp16())
    x = rg.randn([2, 64, 8, 8])
    for _ in range(2):
        sess.run(x)
        prof = sess.last_npu_profile()
        assert len(prof.records) == 7
        for r in prof.records:
            if r.op == "NPU::Flatten":  # a shape change: no kernel
                continue
            assert r.duration_ns > 0 and r.kernel_ns > 0, r
    sess.close()


def test_fused_pool_records_report_zero_time(rg, ref):
    """A conv whose 2x2 max pool runs in its epilogue keeps every op's record
    with the reference's labels; the absorbed pool launches nothing and
    reports 0 ns, and the conv's record carries the pool's time (its kernel
    writes the pooled output)."""
    from rustgears_amd import nn
    rg.manual_seed(29)
    layers = (nn.Sequential().add(nn.Conv2d(3, 16, 3).padding(1)).add(nn.Relu()).add(nn.MaxPool2d(2, 2))
              .add(nn.Flatten()).add(nn.Linear(16 * 16 * 16, 10))).export()
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    x = rg.randn([8, 3, 32, 32])
    y = sess.run(x)
    prof = sess.last_npu_profile()
    assert_bitexact_f32(y, ref.RefProgram(layers).run(x), "int8 conv+pool")
    labels = [r.op for r in prof.records]
    assert labels[1] == "NPU::MaxPool2d(k=2)", labels
    conv, pool = prof.records[0], prof.records[1]
    assert conv.duration_ns > 0 and conv.kernel_ns > 0, conv
    assert pool.duration_ns == 0 and pool.kernel_ns == 0, pool
    sess.close()


def test_first_run_of_a_process_is_not_charged_the_code_object_load():
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import rustgears_amd as rg\n"
        "from rustgears_amd import configs\n"
        "model, x = configs.quickstart()\n"
        "sess = rg.InferenceSession.from_module(model, rg.ExecutionProvider.mi355x_int8())\n"
        "sess.run(x)\n"
        "print(max(r.duration_ns for r in sess.last_npu_profile().records))\n" % ROOT)
    print("[profile] fresh process: first run", flush=True)
    res = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert res.returncode == 0, res.stderr[-2000:]
    worst_ns = int(res.stdout.strip().splitlines()[-1])
    assert worst_ns < 2_000_000, f"first run's slowest op took {worst_ns / 1e3:.1f} us"


def test_mfma_probe_rate_is_positive_and_below_nominal():
    """rgnpu_probe_mfma_rate: the register-only MFMA probe (bench.py
    --workload mfma_peak) runs and reports a rate under the 5.0 POP/s
    nominal i8 peak (2 ops per MAC), for random and zero operands."""
    from rustgears_amd import _native as N
    for rnd in (1, 0):
        ms, tops = ctypes.c_double(), ctypes.c_double()
        N.check(N.lib().rgnpu_probe_mfma_rate(0, 200, rnd, ctypes.byref(ms), ctypes.byref(tops)))
        assert ms.value > 0 and 100.0 < tops.value < 5200.0, (rnd, ms.value, tops.value)
