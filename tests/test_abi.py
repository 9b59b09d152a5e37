"""The C ABI surface, checked without a GPU: libhxmi.so loads, exports every
entry point include/hx.h declares (and nothing else), the ctypes mirrors of
the descriptor structs have the C layout, the config surface enumerates, and
argument errors come back as status codes with a message -- no compute."""
import ctypes
import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "hx.h"


def declared():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(hx_[a-z0-9_]+)\s*\(", text)))


def test_every_declared_symbol_is_exported(hx):
    lib = hx.load()
    names = declared()
    assert len(names) >= 19
    for n in names:
        assert hasattr(lib, n), n
    out = subprocess.run(["nm", "-D", "--defined-only", str(hx._abi.LIB_PATH)], capture_output=True,
                         text=True, check=True).stdout
    exported = sorted(l.split()[-1] for l in out.splitlines() if " T " in l)
    assert exported == names, "the library must export exactly the header's entry points"
    assert set(hx._abi.SIGNATURES) == set(names), "the ctypes binding covers every entry point"


def test_struct_layouts_match_c(hx):
    # MLIR memref descriptor: 2 pointers + offset + sizes[N] + strides[N]
    assert ctypes.sizeof(hx._abi.MemRef2D) == 8 * 7
    assert ctypes.sizeof(hx._abi.MemRef1D) == 8 * 5
    assert hx._abi.MemRef2D.strides.offset == 40
    assert ctypes.sizeof(hx._abi.KernelConfig) == 4 * 11 + 40


def test_build_id_and_error_without_device(hx):
    import torch
    assert "gfx950" in hx.build_id()
    if torch.cuda.is_available():
        pytest.skip("a GPU is visible")
    rc = hx.load().hx_init()
    assert rc == -9  # HX_ERR_NODEVICE
    assert "no HIP device" in hx._abi.last_error()


def test_dtype_errors_are_reported_before_any_launch(hx):
    lib = hx.load()
    m = hx._abi.MemRef2D()
    rc = lib.hx_matmul(ctypes.byref(m), hx._abi.I32, ctypes.byref(m), hx._abi.I32, 0, None, 0, None, 0,
                       ctypes.byref(m), hx._abi.F16, None)
    assert rc == -3 and "hx_matmul" in hx._abi.last_error()
    rc = lib.hx_softmax(ctypes.byref(m), ctypes.byref(m), hx._abi.I8, None)
    assert rc == -3
    rc = lib.hx_gemm_i8(None, None, 0, None, None, None, 99, None)
    assert rc == -3
    rc = lib.hx_weight_release(ctypes.c_void_p(1234))
    assert rc == -8
    rc = lib.hx_config_get(42, 0, None)
    assert rc == -1


def test_config_surface(hx):
    total = 0
    for op in range(1, 12):
        n = hx.config_count(op)
        assert n >= 3
        for i in range(n):
            c = hx.config_get(op, i)
            assert c["op"] == op and c["index"] == i and c["name"]
            assert c["lds_bytes"] <= 160 * 1024, c
            total += 1
    assert total >= 30
    # the three decode-GEMV families (int8, f16, bf16 weights) share one table
    names = [[hx.config_get(op, i)["name"] for i in range(hx.config_count(op))] for op in (6, 7, 8)]
    assert names[0] == names[1] == names[2]
    assert hx.config_get(6, 0)["bk"] == 64 and hx.config_get(7, 0)["bk"] == 32
    # the three row families (softmax, RMSNorm, LayerNorm) share one table:
    # one row per workgroup, then the streaming form at 2, 4, 8 per CU
    rows = [[hx.config_get(op, i) for i in range(hx.config_count(op))] for op in (9, 10, 11)]
    assert [c["name"] for c in rows[0]] == [c["name"] for c in rows[1]] == [c["name"] for c in rows[2]]
    assert [(c["name"], c["col_tiles"]) for c in rows[0]] == [("row", 0), ("stream_2", 2), ("stream_4", 4),
                                                              ("stream_8", 8)]
    with pytest.raises(hx.HXError):
        hx.config_count(12)


def test_missing_library_fails_loudly(hx, monkeypatch, tmp_path):
    monkeypatch.setattr(hx._abi, "_lib", None)
    monkeypatch.setattr(hx._abi, "LIB_PATH", tmp_path / "libhxmi.so")
    with pytest.raises(ImportError, match="no fallback"):
        hx._abi.load()


def test_manifest_without_device(hx):
    """The manifest export needs no GPU: an empty manifest is valid JSON with
    the schema tag, and a too-small buffer is an error that reports the size
    needed."""
    import ctypes
    import json
    L = hx.load()
    prev = L.hx_manifest_enable(0)
    L.hx_manifest_clear()
    doc = hx.manifest()
    assert doc["schema"] == "hx.kernel_manifest/v1" and doc["records"] == []
    assert doc["build"] == hx.build_id()
    need = ctypes.c_size_t(0)
    buf = ctypes.create_string_buffer(8)
    assert hx._abi.ERRORS[L.hx_manifest_json(buf, 8, ctypes.byref(need))] == "HX_ERR_ARG"
    assert need.value > 8 and "needed" in hx._abi.last_error()
    big = ctypes.create_string_buffer(need.value)
    assert L.hx_manifest_json(big, need.value, ctypes.byref(need)) == 0
    assert json.loads(big.value.decode())["records"] == []
    L.hx_manifest_enable(prev)
