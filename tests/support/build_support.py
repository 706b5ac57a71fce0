"""Builds the standalone GPU checker used by tests/test_gpu_devmath.py into
tests/support/_build/ (hipcc, gfx950, same FP flags as the library)."""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
OUT = os.path.join(HERE, "_build")
EXE = os.path.join(OUT, "devmath_gpu_check")


def build() -> str:
    os.makedirs(OUT, exist_ok=True)
    cmd = [os.path.join(os.environ.get("ROCM_PATH", "/opt/rocm"), "bin", "hipcc"), "-O3", "-std=c++17",
           "-ffp-contract=off", "--offload-arch=gfx950", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
           "-o", EXE, os.path.join(HERE, "devmath_gpu_check.hip")]
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"devmath_gpu_check build failed:\n{res.stderr}")
    return EXE


if __name__ == "__main__":
    print(build())
