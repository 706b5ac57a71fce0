"""Builds the standalone GPU programs of the test suite into
tests/support/_build/ (hipcc, gfx950, same FP flags as the library):
devmath_gpu_check (tests/test_gpu_devmath.py), kloop_lab
(tests/test_gpu_kloop_lab.py) and input_quant_lab
(tests/test_gpu_input_quant_lab.py)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build")
EXE = os.path.join(OUT, "devmath_gpu_check")
PROGRAMS = ["devmath_gpu_check", "kloop_lab", "input_quant_lab"]


def build() -> str:
    os.makedirs(OUT, exist_ok=True)
    hipcc = os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc")
    for name in PROGRAMS:
        cmd = [hipcc, "-O3", "-std=c++17", "-ffp-contract=off", "--offload-arch=gfx950", "-Xclang", "-target-feature",
               "-Xclang", "-packed-fp32-ops", "-I", os.path.join(HERE, "..", "..", "include"),
               "-o", os.path.join(OUT, name), os.path.join(HERE, name + ".hip")]
        res = subprocess.run(cmd, capture_output=True, text=True)
        if res.returncode != 0:
            raise RuntimeError(f"{name} build failed:\n{res.stderr}")
    return EXE


if __name__ == "__main__":
    print(build())
