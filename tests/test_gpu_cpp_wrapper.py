"""The C ABI from a C++ caller with no Python and no torch in the process:
tests/cpp/hx_wrapper_driver plays the reference's generated kernel wrapper
(MemRefDescriptors converted to hx descriptors, hipMalloc'd operands, an
explicit stream) and checks each entry point it calls against the CPU oracle
linked into it (tests/cpp/wrapper_driver.cpp)."""
import subprocess
from pathlib import Path

import pytest

DRIVER = Path(__file__).resolve().parent / "cpp" / "hx_wrapper_driver"
CASES = ["matmul_f16_f32_residual_256", "gemm_i8_i32_and_dequant_bitexact_512x384x640",
         "softmax_rmsnorm_64x4096", "resident_w8a16_gemv_4x1376x4096",
         "hx_tune_gemm_i8_512_pin_and_pins_roundtrip", "error_codes"]


def _run():
    assert DRIVER.exists(), "tests/cpp/hx_wrapper_driver is not built: run __graft_entry__.build()"
    return subprocess.run([str(DRIVER)], capture_output=True, text=True, timeout=100)


@pytest.mark.gpu
def test_cpp_wrapper_driver():
    r = _run()
    print(r.stdout)
    assert r.returncode == 0, r.stdout + r.stderr
    for case in CASES:
        assert f"PASS {case}" in r.stdout, r.stdout
    assert "ALL PASS" in r.stdout


def test_cpp_wrapper_driver_refuses_without_a_device():
    """With no GPU the library returns an error from hx_init (no CPU
    fallback); the driver reports it and exits non-zero."""
    import torch
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible: covered by test_cpp_wrapper_driver")
    r = _run()
    assert r.returncode != 0
    assert "FAIL hx_init" in r.stdout and "ALL PASS" not in r.stdout
