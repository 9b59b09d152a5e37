"""Build libhxmi.so (the HIP kernels + C ABI) in-tree for gfx950.

Each translation unit is compiled by hipcc in parallel, then linked into
``hexagon-mlir_amd/libhxmi.so`` with a version script that exports only the
``hx_*`` C entry points declared in ``include/hx.h``.
"""
from __future__ import annotations

import hashlib
import os
import subprocess
import sys
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
OUT = PKG / "libhxmi.so"
OBJDIR = PKG / "_build"
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = "gfx950"

# the GEMM tables are split per operand mode so that their kernel
# instantiations compile in parallel (each takes minutes)
SOURCES = ["hx_gemm_i8.hip", "hx_gemm_w8.hip", "hx_gemm_f16.hip", "hx_gemm_bf16.hip", "hx_gemm.hip",
           "hx_rows.hip", "hx_gemv.hip", "hx_pack.hip", "hx_attn.hip", "hx_api.cpp", "hx_tune.cpp",
           "hx_noalloc.cpp"]

# Packed-FP32 VALU forms are disabled for all device code (they are not
# needed: the hot loops are MFMA or memory bound).  Floating-point
# contraction is off: every product and sum is rounded on its own, as the
# reference arithmetic (and its CPU restatement) specifies -- a fused
# multiply-add, or a multiply fused into its conversion to fp16, rounds once
# and can land one ulp away.
COMMON = ["-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}", "-ffp-contract=off",
          "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
          "-Wno-unused-command-line-argument"]


# Per-file device flags.  The attention kernel keeps MFMA operands and
# results in architectural VGPRs (the score tiles feed VALU softmax code every
# block; in accumulator registers each block would copy them back and forth).
DEVICE_FLAGS = {
    "hx_attn.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form=1"],
}


def source_digest() -> str:
    h = hashlib.sha256()
    files = sorted(CSRC.glob("*")) + [ROOT / "include" / "hx.h", Path(__file__)]
    for f in files:
        if f.is_file():
            h.update(f.name.encode())
            h.update(f.read_bytes())
    return h.hexdigest()[:16]


def _compiler_version() -> str:
    try:
        out = subprocess.run([HIPCC, "--version"], capture_output=True, text=True, check=True).stdout
        for line in out.splitlines():
            if "clang version" in line:
                return line.split("(")[0].strip().replace(" ", "_")
    except Exception:  # noqa: BLE001
        pass
    return "unknown"


def build(verbose: bool = False) -> Path:
    OBJDIR.mkdir(exist_ok=True)
    build_id = f"hxmi-{ARCH}-{source_digest()}-{_compiler_version()}"
    defs = [f'-DHX_BUILD_ID="{build_id}"']

    def compile_one(src: str) -> Path:
        obj = OBJDIR / (src + ".o")
        cmd = [HIPCC, *COMMON, *DEVICE_FLAGS.get(src, []), *defs, "-c", str(CSRC / src), "-o", str(obj)]
        r = subprocess.run(cmd, capture_output=True, text=True)
        if r.returncode != 0:
            sys.stderr.write(r.stdout + r.stderr)
            raise RuntimeError(f"hipcc failed on {src}")
        if verbose:
            sys.stderr.write(r.stderr)
        return obj

    with ThreadPoolExecutor(max_workers=min(len(SOURCES), os.cpu_count() or 4)) as ex:
        objs = list(ex.map(compile_one, SOURCES))

    vscript = OBJDIR / "exports.map"
    vscript.write_text("{ global: hx_*; local: *; };\n")
    tmp = OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs),
           f"-Wl,--version-script={vscript}", "-Wl,--no-undefined", "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("link of libhxmi.so failed")
    os.replace(tmp, OUT)
    return OUT


PROBE_SRC = CSRC / "probe" / "hx_probe.hip"
PROBE_OUT = PKG / "libhxprobe.so"


def build_probe() -> Path:
    """libhxprobe.so: the measurement probes bench.py --ceilings times
    (empty launch, streaming read, copy, MFMA issue); not part of the hx ABI
    and not part of build(): bench.py --ceilings compiles it when it runs."""
    tmp = PROBE_OUT.with_suffix(".so.tmp")
    cmd = [HIPCC, *COMMON, "-shared", str(PROBE_SRC), "-o", str(tmp)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        sys.stderr.write(r.stdout + r.stderr)
        raise RuntimeError("hipcc failed on the probes")
    os.replace(tmp, PROBE_OUT)
    return PROBE_OUT


if __name__ == "__main__":
    print(build(verbose="-v" in sys.argv))
