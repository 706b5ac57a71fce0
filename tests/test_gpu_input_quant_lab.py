"""The input-quantization lab (tests/support/input_quant_lab.hip) on the S
input (8192 x 4096 f32).

Runs a grid-strided read of the input (the read ceiling), a read that holds
16 units per thread, the one-pass shape of the product's input quantization
(one 512-thread workgroup per CU holding 64 units per thread across its
absmax, then quantizing what it holds; no grid barrier), the same with 1024
threads of 32 units, an absmax pass followed by a quantize pass, and a copy
of the input.  Prints
microseconds and TB/s per variant.  Checks that every variant ran and that the
one-pass shape, which must read the whole input before it can store, stays
slower than the plain read of the same bytes.
"""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "support", "_build", "input_quant_lab")


def test_input_quant_lab_runs():
    assert os.path.exists(EXE), "build the lab first (__graft_entry__.build())"
    print("[input_quant_lab] S input, 134 MB", flush=True)
    out = subprocess.run([EXE, "10"], check=True, capture_output=True, text=True, timeout=120).stdout
    print(out, flush=True)
    rows = {l.split()[0]: (float(l.split()[1]), float(l.split()[2])) for l in out.strip().splitlines()}
    assert set(rows) == {"read/stream", "read/hold16", "onepass/8w", "onepass/16w", "twopass", "copy"}
    assert all(us > 0 and tbs > 0 for us, tbs in rows.values())
    # 134 MB at the 8 TB/s nominal peak takes 16.8 us
    assert rows["read/stream"][0] >= 16.0
    assert rows["read/stream"][0] < rows["onepass/8w"][0]
