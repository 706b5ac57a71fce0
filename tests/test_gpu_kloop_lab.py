"""The K-loop lab (tests/support/kloop_lab.hip) on the S layer shape.

Runs the register-only MFMA loop, the same with the per-step barrier and with
the step's LDS fragment reads (with 16x16x64 and with 32x32x32 MFMAs), the
product's DMA-ring K loop (gemm_core.h big_kloop, 4 and 3 stages) and the
MFMA loop with 1-8 independent FMAs per MFMA, and prints microseconds per S layer (274.9 G ops).  Checks that every
variant ran and that the orderings the design relies on hold: taking parts
away never makes the loop slower by more than the run-to-run spread, and
VALU work beyond what overlaps the MFMAs lengthens the loop.
"""
import os
import subprocess

import pytest

from conftest import ROOT

pytestmark = pytest.mark.gpu

EXE = os.path.join(ROOT, "tests", "support", "_build", "kloop_lab")


def test_kloop_lab_runs_and_orders():
    assert os.path.exists(EXE), "build the lab first (__graft_entry__.build())"
    print("[kloop] lab on the S layer shape", flush=True)
    out = subprocess.run([EXE, "10"], check=True, capture_output=True, text=True, timeout=120).stdout
    print(out, flush=True)
    us = {l.split()[0]: float(l.split()[1]) for l in out.strip().splitlines()}
    assert set(us) == {"mfma", "mfma+barrier", "mfma+barrier+lds", "mfma32", "mfma32+barrier",
                       "mfma32+barrier+lds", "production/4", "production/3", "wide/lds",
                       "wide/lds+pf", "overlap/1",
                       "overlap/2", "overlap/3", "overlap/4", "overlap/6", "overlap/8"}
    assert all(v > 0 for v in us.values())
    # 5 POP/s nominal: an S layer cannot take less than 55 us
    assert us["mfma"] >= 54.0
    assert us["mfma"] <= 1.05 * us["mfma+barrier"] and us["mfma+barrier"] <= 1.05 * us["mfma+barrier+lds"]
    assert us["overlap/8"] > us["mfma"]
    assert us["mfma32"] >= 54.0 and us["mfma32"] <= 1.05 * us["mfma32+barrier+lds"]
