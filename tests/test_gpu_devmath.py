"""Exhaustive device check of the branch-free exact activation math.

tests/support/devmath_gpu_check (built by __graft_entry__.build()) evaluates,
on the GPU, the epilogue forms tanhf_fast / gelu_fast and the reference forms
tanhf_fdlibm / gelu for all 2^32 f32 inputs and counts differences.  The
reference forms equal glibc on every input (tests/test_host.py with
RG_EXHAUSTIVE=1, and the device sweep in test_gpu_parity.py).  The same run
checks the certified GELU's bound: |gelu_approx(x) - gelu(x)| <=
kGeluApproxRel |x| + kGeluApproxAbs for every finite f32 x.
"""
import os
import subprocess

import numpy as np
import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "support", "_build", "devmath_gpu_check")


def test_fast_activation_math_equals_reference_on_all_inputs():
    assert os.path.exists(EXE), "build the checker first (__graft_entry__.build())"
    print("[devmath] exhaustive 2^32 device check", flush=True)
    out = subprocess.run([EXE, "1"], check=True, capture_output=True, text=True, timeout=120).stdout
    rows = [l.split() for l in out.strip().splitlines()]
    assert [r[0] for r in rows] == ["tanhf_fast", "gelu_fast", "gelu_approx"]
    for name, checked, bad, first in rows[:2]:
        assert int(checked) == 1 << 32
        assert int(bad) == 0, f"{name}: {bad} inputs differ from the reference form, first 0x{first}"
    name, checked, bad, first, worst = rows[2]
    worst_ratio = np.uint32(int(worst, 16)).view(np.float32)
    print(f"[devmath] gelu_approx: largest |error| / |x| = {worst_ratio:.3e}", flush=True)
    assert int(checked) == (1 << 32) - (1 << 24)  # every finite f32: all patterns but the 2^24 with exponent 255
    assert int(bad) == 0, f"gelu_approx breaks its bound on {bad} inputs, first 0x{first}"
