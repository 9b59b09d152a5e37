"""The plan manifest records, per matmul-family call, the kernel path, the
tile configuration and who chose it, the reason, and how the weight was
supplied (the run-time counterpart of the reference's hmx.kernel_manifest
plan/reason records, QHB/include/hexagon/Dialect/Hmx/Transforms/
HmxManifest.h:81-110)."""
import numpy as np
import pytest
import torch

from conftest import to_dev

pytestmark = pytest.mark.gpu


def records(hx):
    return hx.manifest()["records"]


def test_manifest_records_plans_and_reasons(hx, dev):
    hx.manifest_clear()
    prev = hx.manifest_enable(True)
    try:
        g = torch.Generator(device=dev).manual_seed(5)
        a = torch.randint(-127, 128, (512, 512), dtype=torch.int8, device=dev, generator=g)
        b = torch.randint(-127, 128, (512, 512), dtype=torch.int8, device=dev, generator=g)
        for _ in range(3):
            hx.gemm_i8(a, b, b_layout="nk")                      # aligned -> tiled
        hx.gemm_i8(a, b, b_layout="kn")                          # KN -> read in place (tiled)
        hx.gemm_i8(a, b[:, :504].contiguous(), b_layout="kn")    # KN, N = 504 -> transposed into workspace
        a_tall = torch.randint(-127, 128, (2056, 512), dtype=torch.int8, device=dev, generator=g)
        hx.gemm_i8(a_tall, b, b_layout="kn")                     # KN, M = 2056 -> read in place
        hx.gemm_i8(a[:, :16], b[:, :16], b_layout="nk")          # K=16 bytes -> shallow-k, generic
        hx.gemm_i8(a[:, :112], b[:, :112], b_layout="nk")        # K=112 bytes, shorter than any ring: tiled
        hx.gemm_i8(a[:, :496], b[:36, :496].contiguous(), b_layout="nk")  # strided A, N=36: tiled
        hx.gemm_i8(a[:, :504], b[:36, :504].contiguous(), b_layout="nk")  # ldb=504 -> row-stride
        hx.gemm_i8(a, b[:38].contiguous(), b_layout="nk")         # N=38 -> n-granularity
        x = torch.randn((4, 512), dtype=torch.float16, device=dev, generator=g)
        w = torch.randint(-127, 128, (512, 512), dtype=torch.int8, device=dev, generator=g)
        s = torch.rand(512, device=dev).half()
        hx.gemv_w8a16(x, w, s, w_layout="nk")                    # decode GEMV, weight read in place
        rw = hx.ResidentWeight(w, s, layout="nk")
        try:
            hx.matmul_resident(x, rw)                            # packed decode GEMV
            hx.matmul_resident(torch.randn((32, 512), dtype=torch.float16, device=dev), rw)   # row blocks
            hx.matmul_resident(torch.randn((48, 512), dtype=torch.float16, device=dev), rw)   # tiled
            hx.matmul_resident(torch.randn((128, 512), dtype=torch.float16, device=dev), rw)  # tiled
        finally:
            rw.release()
        # argument f16 weights past 16 rows: row blocks only for a [N][K]
        # weight of >= 2048 columns and <= 24 rows, else the tiled GEMM
        wf = torch.randn((2048, 512), dtype=torch.float16, device=dev, generator=g)
        x20 = torch.randn((20, 512), dtype=torch.float16, device=dev, generator=g)
        hx.matmul(x20, wf, b_layout="nk")                        # row blocks
        hx.matmul(x20, wf.t().contiguous(), b_layout="kn")       # tiled, B read in place
        hx.matmul(x20, wf[:1024], b_layout="nk")                 # N = 1024: tiled
        hx.matmul(torch.randn((40, 512), dtype=torch.float16, device=dev, generator=g), wf, b_layout="nk")
        rf = hx.ResidentWeight(wf, None, layout="nk")           # f16: the packed decode image
        try:
            hx.matmul_resident(torch.randn((3, 512), dtype=torch.float16, device=dev, generator=g), rf)
            hx.matmul_resident(torch.randn((28, 512), dtype=torch.float16, device=dev, generator=g), rf)
        finally:
            rf.release()
        torch.cuda.synchronize()
        recs = records(hx)
    finally:
        hx.manifest_enable(prev)
        hx.manifest_clear()

    def find(**kw):
        got = [r for r in recs if all(r[k] == v for k, v in kw.items())]
        assert got, f"no record with {kw} in {recs}"
        return got[0]

    r = find(entry="hx_gemm_i8", m=512, n=512, k=512, weight="argument", plan="mfma-tiled")
    assert r["calls"] == 3 and r["reason"] == "selected-aligned" and r["config_source"] == "default"
    assert r["a"] == "i8" and r["c"] == "i32"
    assert find(entry="hx_gemm_i8", weight="argument-kn", n=512)["plan"] == "mfma-tiled"
    assert find(entry="hx_gemm_i8", weight="transposed-to-workspace", n=504)["plan"] == "mfma-tiled"
    assert find(entry="hx_gemm_i8", weight="argument-kn", m=2056)["plan"] == "mfma-tiled"
    assert find(entry="hx_gemm_i8", k=16)["reason"] == "shallow-k"
    assert find(entry="hx_gemm_i8", k=16)["plan"] == "mfma-generic"
    assert find(entry="hx_gemm_i8", k=112)["plan"] == "mfma-tiled"
    assert find(entry="hx_gemm_i8", n=38)["reason"] == "n-granularity"
    assert find(entry="hx_gemm_i8", n=36, k=496)["plan"] == "mfma-tiled"
    assert find(entry="hx_gemm_i8", n=36, k=504)["reason"] == "row-stride"  # ldb = 504
    assert find(entry="hx_matmul", m=4, plan="gemv-stream")["reason"] == "min-rows"
    assert find(entry="hx_matmul_resident", m=4)["plan"] == "gemv-packed"
    r = find(entry="hx_matmul_resident", m=32)
    assert r["plan"] == "gemv-packed" and r["reason"] == "few-rows" and r["config"].startswith("rows")
    assert find(entry="hx_matmul_resident", m=48)["plan"] == "mfma-tiled"
    r = find(entry="hx_matmul_resident", m=128)
    assert r["plan"] == "mfma-tiled" and r["weight"] == "resident-image" and r["b"] == "i8"
    r = find(entry="hx_matmul", m=20, n=2048, weight="argument")
    assert r["plan"] == "gemv-stream" and r["reason"] == "few-rows" and r["config"].startswith("rows")
    assert find(entry="hx_matmul", m=20, n=2048, weight="argument-kn")["plan"] == "mfma-tiled"
    assert find(entry="hx_matmul", m=20, n=1024)["plan"] == "mfma-tiled"
    assert find(entry="hx_matmul", m=40, n=2048)["plan"] == "mfma-tiled"
    r = find(entry="hx_matmul_resident", m=3, b="f16")
    assert r["plan"] == "gemv-packed" and r["weight"] == "resident-packed" and r["reason"] == "min-rows"
    r = find(entry="hx_matmul_resident", m=28, b="f16")
    assert r["plan"] == "gemv-packed" and r["reason"] == "few-rows" and r["config"].startswith("rows")


def test_manifest_reports_pinned_config(hx, dev):
    M = N = K = 1024
    a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev)
    b = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
    hx.manifest_clear()
    prev = hx.manifest_enable(True)
    try:
        hx.config_select(1, M, N, K, 3)
        try:
            hx.gemm_i8(a, b, b_layout="nk")
        finally:
            hx.config_select(1, M, N, K, -1)
        hx.gemm_i8(a, b, b_layout="nk")
        torch.cuda.synchronize()
        recs = records(hx)
    finally:
        hx.manifest_enable(prev)
        hx.manifest_clear()
    pinned = [r for r in recs if r["config_source"] == "pinned"]
    default = [r for r in recs if r["config_source"] == "default"]
    assert len(pinned) == 1 and pinned[0]["config"] == hx.config_get(1, 3)["name"]
    assert len(default) == 1
    assert default[0]["config"] == hx.config_get(1, hx.config_lookup(1, M, N, K))["name"]


def test_config_pins_round_trip(hx, dev):
    """Champions survive a save/load round trip; text from another build or
    naming the wrong config is refused and pins nothing."""
    shapes = [(1, 1000, 1000, 1000, 3), (2, 512, 768, 256, 1), (6, 4, 11008, 4096, 2)]
    for op, m, n, k, i in shapes:
        hx.config_select(op, m, n, k, i)
    text = hx.config_pins_save()
    assert text.startswith("hx-pins/v2 " + hx.build_id())
    for op, m, n, k, i in shapes:
        hx.config_select(op, m, n, k, -1)
    try:
        hx.config_pins_load(text)
        for op, m, n, k, i in shapes:
            assert hx.config_lookup(op, m, n, k) == i
        for op, m, n, k, i in shapes:
            hx.config_select(op, m, n, k, -1)
        before = hx.config_pins_save()
        other = text.replace(hx.build_id(), "hxmi-gfx950-0000000000000000-x", 1)
        with pytest.raises(hx.HXError, match="pins are from"):
            hx.config_pins_load(other)
        wrong = text.splitlines()[0] + "\npin 1 1000 1000 1000 3 not_a_config\n"
        with pytest.raises(hx.HXError, match="is not config"):
            hx.config_pins_load(wrong)
        assert hx.config_pins_save() == before, "a refused load must pin nothing"
    finally:
        for op, m, n, k, i in shapes:
            hx.config_select(op, m, n, k, -1)
