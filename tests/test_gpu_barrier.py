"""The persistent grids' barrier (fused requantization, one-pass input
quantization): its counters and the cost of one poll.

* On one stream every workgroup of a grid is resident: no workgroup defers
  and none is ever found unsettled; every barrier launch is counted.
* With RGNPU_REQUANT_SPIN_LIMIT=0 every workgroup but the finisher defers,
  the results stay bit-exact, and nothing is unsettled.
* Runs from several host threads on one session (worker streams, each with
  its own grids that each fill the GPU) stay bit-identical to the serial
  result, and none of their workgroups defers: worker streams order their
  persistent grids.
* One poll's cost (rgnpu_probe_barrier_poll) is what the wait bound's
  documentation states (kBarrierPollUs).
"""
import ctypes
import threading

import numpy as np
import pytest

from conftest import assert_bitexact_f32

pytestmark = pytest.mark.gpu


def _stack(rg, width=2048, depth=3, rows=4096, seed=17):
    from rustgears_amd import nn
    rg.manual_seed(seed)
    m = nn.Sequential()
    for _ in range(depth):
        m.add(nn.Linear(width, width)).add(nn.Gelu())
    return m.export(), rg.randn([rows, width])


def test_barrier_counters_on_one_stream(rg, ref):
    layers, x = _stack(rg)
    print("[barrier] one stream, 3 x 2048^2 GELU, 4096 rows", flush=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    first = sess.barrier_stats()
    y2 = sess.run(x)
    second = sess.barrier_stats()
    sess.close()
    want = ref.RefProgram(layers).run(x, parallel=True)
    assert_bitexact_f32(y, want, "run 1")
    assert_bitexact_f32(y2, want, "run 2")
    # the input quantization and the two fused requantizations
    assert first == {"deferred": 0, "unsettled": 0, "launches": 3}, first
    assert second == {"deferred": 0, "unsettled": 0, "launches": 6}, second


def test_barrier_counters_with_forced_deferral(rg, ref, monkeypatch):
    monkeypatch.setenv("RGNPU_REQUANT_SPIN_LIMIT", "0")
    layers, x = _stack(rg)
    print("[barrier] spin limit 0", flush=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    y = sess.run(x)
    st = sess.barrier_stats()
    sess.close()
    assert_bitexact_f32(y, ref.RefProgram(layers).run(x, parallel=True), "deferred")
    assert st["launches"] == 3 and st["unsettled"] == 0 and st["deferred"] > 0, st
    print(f"[barrier] forced: {st}", flush=True)


def test_barrier_counters_under_concurrent_runs(rg, ref):
    """8192 rows of 2048-wide layers: 256 tiles of 256 x 256, so every
    persistent grid asks for the whole GPU.  Once two host runs of a session
    have overlapped, its worker runs use the plans without persistent grids
    (program.cpp make_plan), so after a first concurrent round nothing
    launches a barrier grid and nothing defers; every output stays
    bit-identical to the serial result."""
    layers, x = _stack(rg, rows=8192)
    want = ref.RefProgram(layers).run(x, parallel=True)
    sess = rg.InferenceSession.from_layers(layers, rg.ExecutionProvider.mi355x_int8())
    errors = []

    def rounds(k, n):
        try:
            for _ in range(n):
                y = sess.run(x)
                if not np.array_equal(y.view(np.uint32), want.view(np.uint32)):
                    errors.append(f"thread {k}: output differs")
        except Exception as e:  # noqa: BLE001 -- reported below
            errors.append(f"thread {k}: {e}")

    def threads(n):
        ts = [threading.Thread(target=rounds, args=(k, n)) for k in range(4)]
        for t in ts:
            t.start()
        for t in ts:
            t.join()

    print("[barrier] 4 threads x 2 runs, then 4 threads x 6 runs on one session", flush=True)
    threads(2)
    first = sess.barrier_stats()
    threads(6)
    st = sess.barrier_stats()
    sess.close()
    assert not errors, errors
    assert st["unsettled"] == 0, st
    assert st["launches"] == first["launches"] and st["deferred"] == first["deferred"], (first, st)
    print(f"[barrier] concurrent: first round {first}, after {st}", flush=True)


def test_barrier_poll_cost(rg):
    us = ctypes.c_double()
    rg._native.check(rg.lib().rgnpu_probe_barrier_poll(0, 256, 20000, ctypes.byref(us)))
    print(f"[barrier] one poll: {us.value:.3f} us (256 workgroups)", flush=True)
    # the documented figure (kBarrierPollUs = 0.32 us) within a factor of 2
    assert 0.16 <= us.value <= 0.64, us.value
