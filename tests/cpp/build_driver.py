"""Build tests/cpp/hx_wrapper_driver: the C++ caller of libhxmi (no Python,
no torch) with the CPU oracle linked in as its checker.  Called by
__graft_entry__.build() after libhxmi.so is built; the GPU test only runs
the binary."""
from __future__ import annotations

import os
import subprocess
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parent.parent
OUT = HERE / "hx_wrapper_driver"
ROCM = os.environ.get("ROCM_PATH", "/opt/rocm")


def build() -> Path:
    obj_dir = HERE / "_build"
    obj_dir.mkdir(exist_ok=True)
    oracle_obj = obj_dir / "hx_oracle.o"
    cmds = [
        ["gcc", "-O2", "-fPIC", "-ffp-contract=off", "-fno-math-errno", "-c",
         str(ROOT / "oracle" / "hx_oracle.c"), "-o", str(oracle_obj)],
        # host code only (no kernels): g++ with the HIP runtime's headers and
        # library; the rpath finds libhxmi.so in the package directory
        ["g++", "-O2", "-std=c++17", "-D__HIP_PLATFORM_AMD__", "-I", str(ROOT / "include"),
         "-I", f"{ROCM}/include", str(HERE / "wrapper_driver.cpp"), str(oracle_obj),
         "-L", str(ROOT / "hexagon-mlir_amd"), "-lhxmi", "-L", f"{ROCM}/lib", "-lamdhip64",
         f"-Wl,-rpath,$ORIGIN/../../hexagon-mlir_amd:{ROCM}/lib", "-o", str(OUT) + ".tmp"],
    ]
    for cmd in cmds:
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"build of the C++ wrapper driver failed: {cmd[0]}")
    os.replace(str(OUT) + ".tmp", OUT)
    return OUT


if __name__ == "__main__":
    print(build())
