"""GPU parity for the MFMA GEMM family.

int8 x int8 -> int32 is compared BIT-EXACT with the oracle (integer sums are
order-free); the fused dequant to fp16 is bit-exact too (the epilogue computes
RNE_f16(((float)acc * sa) * sb) in the same binary32 order).  Floating GEMMs
are within rtol 1e-2 / atol 1e-3 of the oracle, and additionally under the
reference's own relative-Frobenius gate rel < 2e-3 against an f32 product
(test/python/triton/test_matmul_kloop.py:68, test_matmul_multispan.py:69).
At the full 4096^3 size, exactness is checked on sampled rows plus the
size-independent identities colsum(C) = colsum(A).B and C.1 = A.(B.1).
"""
import numpy as np
import pytest

from conftest import assert_close, bf16_from_f32, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu


def i8(shape, seed):
    return rng(seed).integers(-127, 128, shape, dtype=np.int8)


def rel_fro(got, want):
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    return np.linalg.norm(got - want) / np.linalg.norm(want)


I8_SHAPES = [(256, 256, 256), (128, 256, 512), (100, 72, 48), (64, 80, 160), (1, 300, 4096),
             (333, 257, 96), (17, 33, 50), (513, 1030, 4112)]


@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("shape", I8_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_gemm_i8_exact(hx, dev, shape, layout):
    M, N, K = shape
    a = i8((M, K), 1)
    b = i8((K, N), 2)
    bt = np.ascontiguousarray(b.T)
    c = hx.gemm_i8(to_dev(a, dev), to_dev(b if layout == "kn" else bt, dev), b_layout=layout)
    want = oracle.gemm_i8_i32(a, b)
    got = to_np(c)
    assert np.array_equal(got, want), f"int8 GEMM {shape} {layout}: {int((got != want).sum())} differ"


@pytest.mark.parametrize("shape", [(256, 256, 256), (300, 500, 4096), (64, 64, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemm_i8_dequant_f16_bitexact(hx, dev, shape):
    M, N, K = shape
    a, b = i8((M, K), 3), i8((K, N), 4)
    sa = rng(5).uniform(0.001, 0.02, M).astype(np.float32)
    sb = rng(6).uniform(0.001, 0.02, N).astype(np.float32)
    import torch
    c = hx.gemm_i8(to_dev(a, dev), to_dev(b, dev), row_scale=to_dev(sa, dev), col_scale=to_dev(sb, dev),
                   out_dtype=torch.float16)
    want = oracle.dequant_i32_f16(oracle.gemm_i8_i32(a, b), sa, sb)
    got = to_np(c)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), \
        f"dequant differs in {int((got.view(np.uint16) != want.view(np.uint16)).sum())} elements"


@pytest.mark.parametrize("which", ["row", "col", "none"])
@pytest.mark.parametrize("shape", [(300, 260, 512), (256, 256, 256)], ids=lambda s: "x".join(map(str, s)))
def test_gemm_i8_one_sided_scales(hx, dev, shape, which):
    """Dequant with only the row scale, only the column scale, or neither: an
    absent scale multiplies by nothing (the epilogue multiplies by 1.0, which is
    exact), so each case is bit-exact against the oracle's own one-sided form."""
    import torch
    M, N, K = shape
    a, b = i8((M, K), 31), i8((K, N), 32)
    sa = rng(33).uniform(0.001, 0.02, M).astype(np.float32) if which == "row" else None
    sb = rng(34).uniform(0.001, 0.02, N).astype(np.float32) if which == "col" else None
    c = hx.gemm_i8(to_dev(a, dev), to_dev(b, dev),
                   row_scale=None if sa is None else to_dev(sa, dev),
                   col_scale=None if sb is None else to_dev(sb, dev), out_dtype=torch.float16)
    want = oracle.dequant_i32_f16(oracle.gemm_i8_i32(a, b), sa, sb)
    got = to_np(c)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16)), \
        f"{which}: {int((got.view(np.uint16) != want.view(np.uint16)).sum())} differ"


@pytest.mark.parametrize("out", ["f32", "bf16"])
def test_gemm_i8_dequant_wide_and_bf16_out(hx, dev, out):
    """The dequant epilogue's other output types: ((float)acc * sa[i]) * sb[j]
    in binary32 (numpy float32 products round the same way), stored as f32 or
    rounded to bf16 (RNE) -- bit-exact either way."""
    import torch
    M, N, K = 272, 392, 640
    a, b = i8((M, K), 35), i8((K, N), 36)
    sa = rng(37).uniform(0.001, 0.02, M).astype(np.float32)
    sb = rng(38).uniform(0.001, 0.02, N).astype(np.float32)
    c = hx.gemm_i8(to_dev(a, dev), to_dev(b, dev), row_scale=to_dev(sa, dev), col_scale=to_dev(sb, dev),
                   out_dtype=torch.float32 if out == "f32" else torch.bfloat16)
    acc = oracle.gemm_i8_i32(a, b).astype(np.float32)
    want32 = (acc * sa[:, None]) * sb[None, :]
    got = to_np(c)
    if out == "f32":
        assert np.array_equal(got.view(np.uint32), want32.view(np.uint32))
    else:
        assert np.array_equal(got, bf16_from_f32(want32))


def test_gemm_i8_extremes_closed_form(hx, dev):
    """All +127 times all -127: every entry is -K*127^2 (no int32 overflow
    at K=4096: 66,064,384 < 2^31); identity B reproduces A exactly."""
    K = 4096
    a = np.full((64, K), 127, np.int8)
    b = np.full((K, 96), -127, np.int8)
    c = to_np(hx.gemm_i8(to_dev(a, dev), to_dev(b, dev)))
    assert (c == -K * 127 * 127).all()
    a2 = i8((128, 256), 7)
    eye = np.eye(256, dtype=np.int8)
    c2 = to_np(hx.gemm_i8(to_dev(a2, dev), to_dev(eye, dev)))
    assert np.array_equal(c2, a2.astype(np.int32))


def test_gemm_i8_4096_cube(hx, dev):
    """BASELINE config C2 at full size: the whole 4096 x 4096 int32 output and
    the whole fused-dequant fp16 output bit-exact against the oracle (which
    computes the full product on the host's threads), plus the exact
    column/row checksum identities as an independent check of the oracle."""
    import torch
    M = N = K = 4096
    a = i8((M, K), 11)
    b = i8((K, N), 12)
    bt = np.ascontiguousarray(b.T)
    c = hx.gemm_i8(to_dev(a, dev), to_dev(bt, dev), b_layout="nk")
    got = to_np(c)
    want = oracle.gemm_i8_i32(a, b)
    bad = got != want
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} int32 outputs differ, first at {np.argwhere(bad)[:3].tolist()}"
    a64, b64 = a.astype(np.int64), b.astype(np.int64)
    assert np.array_equal(got.astype(np.int64).sum(axis=0), a64.sum(axis=0) @ b64), "column checksums"
    assert np.array_equal(got.astype(np.int64).sum(axis=1), a64 @ b64.sum(axis=1)), "row checksums"
    # the fused-dequant output of the same product, every element bit-exact
    sa = rng(14).uniform(0.001, 0.02, M).astype(np.float32)
    sb = rng(15).uniform(0.001, 0.02, N).astype(np.float32)
    c16 = hx.gemm_i8(to_dev(a, dev), to_dev(bt, dev), b_layout="nk", row_scale=to_dev(sa, dev),
                     col_scale=to_dev(sb, dev), out_dtype=torch.float16)
    want16 = oracle.dequant_i32_f16(want, sa, sb)
    bad16 = to_np(c16).view(np.uint16) != want16.view(np.uint16)
    assert not bad16.any(), f"{int(bad16.sum())} fp16 outputs differ"


N_I8_CONFIGS = 18


@pytest.mark.parametrize("K", [1024, 1072, 1152, 208, 144, 112, 32])
@pytest.mark.parametrize("cfg", range(N_I8_CONFIGS))
def test_gemm_i8_every_config(hx, dev, cfg, K):
    """Every compiled int8 configuration is exact (the autotuner may pick
    any): edge tiles in M and N, K stage counts that leave each remainder of
    the three-stage ring (1072 = 16.75 stages of 64 bytes, 1152 = 18), K
    shorter than the stage ring (208, 144), shorter than one stage (112, and
    32: a single MFMA k-step) and, for the split configs, parts of unequal
    length."""
    assert hx.config_count(1) == N_I8_CONFIGS, "new int8 configs: extend this test's range"
    M, N = 384, 640
    a, b = i8((M, K), 20), i8((K, N), 21)
    hx.config_select(1, M, N, K, cfg)
    try:
        got = to_np(hx.gemm_i8(to_dev(a, dev), to_dev(np.ascontiguousarray(b.T), dev), b_layout="nk"))
    finally:
        hx.config_select(1, M, N, K, -1)
    assert np.array_equal(got, oracle.gemm_i8_i32(a, b)), hx.config_get(1, cfg)["name"]


@pytest.mark.parametrize("shape", [(384, 640, 1024), (200, 144, 272), (64, 2048, 4096)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemm_i8_kn_in_place_every_config(hx, dev, shape):
    """int8 B in the linalg [K][N] orientation read in place by the tiled
    kernel (transposing 8-bit LDS reads, no transposed copy): every config
    bit-exact, edge tiles and a K tail included, and the fused dequant."""
    import torch
    M, N, K = shape
    a, b = i8((M, K), 160), i8((K, N), 161)
    want = oracle.gemm_i8_i32(a, b)
    ad, bd = to_dev(a, dev), to_dev(b, dev)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        for cfg in range(hx.config_count(1)):
            hx.config_select(1, M, N, K, cfg)
            try:
                got = to_np(hx.gemm_i8(ad, bd, b_layout="kn"))
            finally:
                hx.config_select(1, M, N, K, -1)
            assert np.array_equal(got, want), hx.config_get(1, cfg)["name"]
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    assert recs and all(r["weight"] == "argument-kn" and r["plan"] == "mfma-tiled" for r in recs), recs
    sa = rng(162).uniform(0.001, 0.02, M).astype(np.float32)
    sb = rng(163).uniform(0.001, 0.02, N).astype(np.float32)
    c = hx.gemm_i8(ad, bd, b_layout="kn", row_scale=to_dev(sa, dev), col_scale=to_dev(sb, dev),
                   out_dtype=torch.float16)
    assert np.array_equal(to_np(c).view(np.uint16), oracle.dequant_i32_f16(want, sa, sb).view(np.uint16))


@pytest.mark.parametrize("out", ["i32", "f16", "bf16", "f32"])
@pytest.mark.parametrize("name", ["256x256_w2x4_k2", "128x128_w2x2_k2", "64x64_w2x2_k4"])
def test_gemm_i8_split_k_dequant_bitexact(hx, dev, name, out):
    """int8 K split: int32 partials summed with wrap-around equal the
    unsplit accumulator, and the merge's dequant ((acc * row) * col, one
    rounding to the output type) equals the fused epilogue's bit for bit;
    one-sided and two-sided scales, K not a multiple of the part size."""
    import torch
    M, N, K = 272, 200, 1936
    a, bt = i8((M, K), 150), i8((N, K), 151)
    sa = rng(152).uniform(0.001, 0.02, M).astype(np.float32)
    sb = rng(153).uniform(0.001, 0.02, N).astype(np.float32)
    names = [hx.config_get(1, i)["name"] for i in range(hx.config_count(1))]
    cfg = names.index(name)
    assert hx.config_get(1, cfg)["split_k"] > 1
    acc = oracle.gemm_i8_i32(a, bt, b_trans=True)
    tdt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}
    hx.config_select(1, M, N, K, cfg)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        ad, bd = to_dev(a, dev), to_dev(bt, dev)
        if out == "i32":
            got = to_np(hx.gemm_i8(ad, bd, b_layout="nk"))
            assert np.array_equal(got, acc)
        else:
            for rs, cs in ((sa, sb), (sa, None), (None, sb)):
                c = hx.gemm_i8(ad, bd, b_layout="nk", row_scale=None if rs is None else to_dev(rs, dev),
                               col_scale=None if cs is None else to_dev(cs, dev), out_dtype=tdt[out])
                ones_m, ones_n = np.ones(M, np.float32), np.ones(N, np.float32)
                v = (acc.astype(np.float32) * (ones_m if rs is None else rs)[:, None]) * \
                    (ones_n if cs is None else cs)[None, :]
                if out == "f16":
                    want = oracle.dequant_i32_f16(acc, rs, cs)
                    assert np.array_equal(to_np(c).view(np.uint16), want.view(np.uint16))
                elif out == "bf16":
                    got = to_np(c.view(torch.int16)).view(np.uint16)
                    assert np.array_equal(got, bf16_from_f32(v).view(np.uint16))
                else:
                    assert np.array_equal(to_np(c).view(np.uint32), v.view(np.uint32))
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
        hx.config_select(1, M, N, K, -1)
    assert recs and all(r["config"] == name for r in recs), recs


def _fp(dtype, shape, seed, lo=-1.0, hi=1.0):
    x = rng(seed).uniform(lo, hi, shape).astype(np.float32)
    if dtype == "f16":
        return x.astype(np.float16)
    return bf16_from_f32(x)


def _torch(h, dtype, dev):
    import torch
    if dtype == "bf16":
        return to_dev(h.view(np.int16), dev).view(torch.bfloat16)
    return to_dev(h, dev)


def _vals(h, dtype):
    return oracle.bf16_bits_to_f32(h) if dtype == "bf16" else np.asarray(h, np.float32)


F_SHAPES = [(256, 256, 256), (256, 256, 512), (1024, 512, 64), (256, 64, 2048), (128, 128, 128), (100, 200, 72),
            (33, 65, 17), (512, 384, 1024)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("shape", F_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_matmul_float(hx, dev, dtype, layout, shape):
    M, N, K = shape
    a = _fp(dtype, (M, K), 30)
    b = _fp(dtype, (K, N), 31)
    bb = b if layout == "kn" else np.ascontiguousarray(b.T)
    c = hx.matmul(_torch(a, dtype, dev), _torch(bb, dtype, dev), b_layout=layout)
    bf = dtype == "bf16"
    want = oracle.matmul(a, b, a_bf16=bf, b_bf16=bf, out_bf16=bf)
    rtol, atol = (1e-2, 1e-3) if dtype == "f16" else (2e-2, 1e-2)
    got = _vals(to_np(c), dtype)
    assert_close(got, _vals(want, dtype), rtol, atol, f"matmul {dtype} {shape} {layout}")
    exact = _vals(a, dtype).astype(np.float64) @ _vals(b, dtype).astype(np.float64)
    assert rel_fro(got, exact) < (2e-3 if dtype == "f16" else 8e-3)


def test_matmul_multispan_output_stride(hx, dev):
    """The multi-span ABI: a 2048^3 product written into a window of a wider
    output (row stride 2304), as test/python/triton/test_matmul_multispan.py
    exercises; nothing outside the window may change, rel < 2e-3."""
    import torch
    M = N = K = 2048
    a = _fp("f16", (M, K), 40, 0.0, 1.0)
    b = _fp("f16", (K, N), 41, 0.0, 1.0)
    big = torch.full((M, N + 256), -3.0, dtype=torch.float16, device=dev)
    hx.matmul(to_dev(a, dev), to_dev(b, dev), out=big[:, :N])
    got = to_np(big)
    assert (got[:, N:] == np.float16(-3.0)).all()
    exact = a.astype(np.float64) @ b.astype(np.float64)
    assert rel_fro(got[:, :N], exact) < 2e-3


def test_matmul_residual_scale_f32_out(hx, dev):
    """C = A.B * col_scale + residual, f32 out (the widened read-out with a
    residual, QHB/bin/runtime/hmx/src/HMXLayout.c:868-999)."""
    import torch
    M, N, K = 192, 320, 256
    a, b = _fp("f16", (M, K), 50), _fp("f16", (K, N), 51)
    r = rng(52).normal(0, 1, (M, N)).astype(np.float32)
    s = rng(53).uniform(0.5, 2.0, N).astype(np.float32)
    c = hx.matmul(to_dev(a, dev), to_dev(b, dev), col_scale=to_dev(s, dev), residual=to_dev(r, dev),
                  out_dtype=torch.float32)
    want = oracle.matmul(a, b, scale_n=s, residual=r, out_dtype=np.float32)
    assert_close(to_np(c), want, 1e-4, 1e-4, "residual+scale f32")
    # dropping either term is caught
    assert not np.allclose(to_np(c), oracle.matmul(a, b, residual=r, out_dtype=np.float32), atol=1e-3)
    assert not np.allclose(to_np(c), oracle.matmul(a, b, scale_n=s, out_dtype=np.float32), atol=1e-3)


@pytest.mark.parametrize("segments", [2, 4])
def test_matmul_k_looped_accumulator(hx, dev, segments):
    """The K-looped form of test/python/triton/test_matmul_kloop.py:73-95:
    M = N = 256, K = 512 walked in BLOCK_K segments with one f32 accumulator
    carried across them.  Each segment is one hx_matmul whose residual and
    output are the same f32 tensor (the read-out lands in the resident
    accumulator, MatmulToHmxPass.cpp:1237-1305); the last segment writes the
    f16 result directly.  Gate: rel < 2e-3 against the f64 product (:67), and
    every segment must take the MFMA tile path with no fallback (:127-130)."""
    import torch
    M = N = 256
    K = 512
    bk = K // segments
    g = torch.Generator().manual_seed(0)
    a = torch.rand((M, K), generator=g).to(torch.float16)
    b = torch.rand((K, N), generator=g).to(torch.float16)
    ad, bd = a.to(dev), b.to(dev)
    acc = torch.full((M, N), float("nan"), dtype=torch.float32, device=dev)
    out = torch.empty((M, N), dtype=torch.float16, device=dev)
    hx.manifest_clear()
    hx.manifest_enable(True)
    try:
        for s in range(segments):
            a_seg, b_seg = ad[:, s * bk:(s + 1) * bk], bd[s * bk:(s + 1) * bk, :]
            last = s == segments - 1
            hx.matmul(a_seg, b_seg, residual=acc if s else None, out=out if last else acc)
        records = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    exact = a.double().numpy() @ b.double().numpy()
    assert rel_fro(to_np(out), exact) < 2e-3
    assert sum(r["calls"] for r in records) == segments
    assert {(r["plan"], r["reason"]) for r in records} == {("mfma-tiled", "selected-aligned")}
    # the carried accumulator holds the f32 sum of all but the last segment
    part = a[:, :K - bk].double().numpy() @ b[:K - bk, :].double().numpy()
    assert rel_fro(to_np(acc), part) < 1e-5


@pytest.mark.parametrize("shape", [(512, 1024, 512), (2048, 704, 4096), (40, 96, 64), (77, 130, 48)],
                         ids=lambda s: "x".join(map(str, s)))
def test_matmul_w8a16_gemm(hx, dev, shape):
    """f16 activations x int8 weights (per-channel f16 scales), M > 16 GEMM."""
    M, N, K = shape
    x = rng(60).normal(0, 1, (M, K)).astype(np.float16)
    w = i8((K, N), 61)
    s = rng(62).uniform(0.001, 0.02, N).astype(np.float16)
    y = hx.matmul(to_dev(x, dev), to_dev(w, dev), col_scale=to_dev(s, dev))
    want = oracle.matmul(x, w, scale_n=s.astype(np.float32))
    assert_close(to_np(y).astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, f"w8a16 {shape}")


@pytest.mark.parametrize("K", [512, 64, 16])
@pytest.mark.parametrize("op", [2, 4])
def test_float_every_config(hx, dev, op, K):
    """Every f16 and W8A16 configuration, incl. K shorter than one stage
    (64) and equal to one k-step (16); the ring runs its extra stages on zero fill."""
    M, N = 320, 448
    a = _fp("f16", (M, K), 70)
    if op == 2:
        b = _fp("f16", (N, K), 71)
        want = oracle.matmul(a, b, b_trans=True)
    else:
        b = i8((N, K), 71)
        want = oracle.matmul(a, b, b_trans=True)
    for cfg in range(hx.config_count(op)):
        hx.config_select(op, M, N, K, cfg)
        try:
            got = to_np(hx.matmul(to_dev(a, dev), to_dev(b, dev), b_layout="nk"))
        finally:
            hx.config_select(op, M, N, K, -1)
        assert_close(got.astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, f"op {op} cfg {cfg}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(320, 448, 512), (200, 136, 264), (96, 1024, 192)],
                         ids=lambda s: "x".join(map(str, s)))
def test_matmul_kn_in_place_every_config(hx, dev, dtype, shape):
    """[K][N] (linalg orientation) f16 / bf16 B read in place by the tiled
    kernel (transposing LDS reads, no transposed copy), every config, edge
    tiles included; with a column scale and an f32 residual once."""
    import torch
    M, N, K = shape
    a = _fp(dtype, (M, K), 130)
    b = _fp(dtype, (K, N), 131)
    bf = dtype == "bf16"
    want = oracle.matmul(a, b, a_bf16=bf, b_bf16=bf, out_bf16=bf)
    rtol, atol = (1e-2, 1e-3) if dtype == "f16" else (2e-2, 1e-2)
    op = 2 if dtype == "f16" else 3
    ad, bd = _torch(a, dtype, dev), _torch(b, dtype, dev)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        for cfg in range(hx.config_count(op)):
            hx.config_select(op, M, N, K, cfg)
            try:
                got = _vals(to_np(hx.matmul(ad, bd, b_layout="kn")), dtype)
            finally:
                hx.config_select(op, M, N, K, -1)
            assert_close(got, _vals(want, dtype), rtol, atol, f"kn {dtype} {shape} cfg {cfg}")
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    assert recs and all(r["weight"] == "argument-kn" and r["plan"] == "mfma-tiled" for r in recs), recs
    s = rng(132).uniform(0.5, 1.5, N).astype(np.float32)
    r = rng(133).normal(0, 1, (M, N)).astype(np.float32)
    c = hx.matmul(ad, bd, b_layout="kn", col_scale=to_dev(s, dev), residual=to_dev(r, dev),
                  out_dtype=torch.float32)
    want32 = oracle.matmul(a, b, a_bf16=bf, b_bf16=bf, scale_n=s, residual=r, out_dtype=np.float32)
    assert_close(to_np(c), want32, 1e-4, 1e-4, f"kn scaled residual {dtype} {shape}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("layout", ["nk", "kn"])
def test_matmul_split_k_scale_residual(hx, dev, dtype, layout):
    """The K-split config (binary32 partials over two K parts, merged with
    the column scale and the residual) against the oracle, with K not a
    multiple of the part size and an edge tile."""
    import torch
    M, N, K = 272, 200, 1000
    a = _fp(dtype, (M, K), 140)
    b = _fp(dtype, (K, N), 141)
    bf = dtype == "bf16"
    s = rng(142).uniform(0.5, 1.5, N).astype(np.float32)
    r = rng(143).normal(0, 1, (M, N)).astype(np.float32)
    op = 2 if dtype == "f16" else 3
    names = [hx.config_get(op, i)["name"] for i in range(hx.config_count(op))]
    cfg = names.index("256x256_w2x4_k2")
    bb = b if layout == "kn" else np.ascontiguousarray(b.T)
    hx.config_select(op, M, N, K, cfg)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        c = hx.matmul(_torch(a, dtype, dev), _torch(bb, dtype, dev), b_layout=layout,
                      col_scale=to_dev(s, dev), residual=to_dev(r, dev), out_dtype=torch.float32)
        plain = hx.matmul(_torch(a, dtype, dev), _torch(bb, dtype, dev), b_layout=layout)
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
        hx.config_select(op, M, N, K, -1)
    assert all(rc["config"] == "256x256_w2x4_k2" for rc in recs), recs
    want = oracle.matmul(a, b, a_bf16=bf, b_bf16=bf, scale_n=s, residual=r, out_dtype=np.float32)
    assert_close(to_np(c), want, 1e-4, 1e-4, f"split-K {dtype} {layout}")
    want16 = oracle.matmul(a, b, a_bf16=bf, b_bf16=bf, out_bf16=bf)
    rtol, atol = (1e-2, 1e-3) if dtype == "f16" else (2e-2, 1e-2)
    assert_close(_vals(to_np(plain), dtype), _vals(want16, dtype), rtol, atol, f"split-K plain {dtype} {layout}")


@pytest.mark.parametrize("dtype,res_dtype", [("f16", "f16"), ("bf16", "bf16"), ("f16", "f32"), ("bf16", "f16")])
def test_matmul_split_k_merge_widths_agree(hx, dev, dtype, res_dtype):
    """The K-split merge runs eight columns per thread when the output and
    residual row strides are multiples of 8 and four otherwise.  The same
    partials merged both ways (outputs with row strides 200 and 204) agree
    bit for bit, with the column scale, a residual of another type and a
    rounded 16-bit output, and match the oracle."""
    import torch
    M, N, K = 272, 200, 1000
    a = _fp(dtype, (M, K), 150)
    b = _fp(dtype, (N, K), 151)
    bf = dtype == "bf16"
    s = rng(152).uniform(0.5, 1.5, N).astype(np.float32)
    r = rng(153).normal(0, 1, (M, N)).astype(np.float32)
    tdt = torch.bfloat16 if bf else torch.float16
    rt = {"f16": torch.float16, "bf16": torch.bfloat16, "f32": torch.float32}[res_dtype]
    op = 2 if dtype == "f16" else 3
    names = [hx.config_get(op, i)["name"] for i in range(hx.config_count(op))]
    hx.config_select(op, M, N, K, names.index("256x256_w2x4_k2"))
    try:
        A, B = _torch(a, dtype, dev), _torch(b, dtype, dev)
        res8 = torch.from_numpy(r).to(dev).to(rt)
        res4 = torch.zeros((M, 204), dtype=rt, device=dev)[:, :N]
        res4.copy_(res8)
        outs = []
        for ld, res in ((200, res8), (204, res4)):
            out = torch.full((M, ld), 7.0, dtype=tdt, device=dev)[:, :N]
            hx.matmul(A, B, b_layout="nk", col_scale=to_dev(s, dev), residual=res, out=out)
            outs.append(out.contiguous().view(torch.int16).cpu())
        torch.cuda.synchronize()
    finally:
        hx.config_select(op, M, N, K, -1)
    assert torch.equal(outs[0], outs[1])
    rq = res8.float().cpu().numpy()
    want = oracle.matmul(a, np.ascontiguousarray(b.T), a_bf16=bf, b_bf16=bf, scale_n=s, residual=rq,
                         out_dtype=np.float32)
    got = outs[0].numpy().view(np.uint16)
    got = oracle.bf16_bits_to_f32(got) if bf else got.view(np.float16).astype(np.float32)
    rtol, atol = (1e-2, 1e-2) if not bf else (2e-2, 5e-2)
    assert_close(got, want, rtol, atol, f"split-K merge {dtype} res {res_dtype}")


@pytest.mark.parametrize("cfg_name", ["256x256_w2x4_k2", "128x128_w2x2_k2", "64x64_w2x2_k4"])
def test_matmul_w8a16_split_k_scale_residual(hx, dev, cfg_name):
    """W8A16 (f16 activations, int8 [N][K] weights) through each K-split
    config, with the per-channel f16 scale and an f16 residual merged after
    the partial sums: an edge tile in M and N, and K not a multiple of the
    part size."""
    import torch
    M, N, K = 200, 328, 1168
    x = rng(160).normal(0, 1, (M, K)).astype(np.float16)
    w = i8((N, K), 161)
    s = rng(162).uniform(0.001, 0.02, N).astype(np.float16)
    r = rng(163).normal(0, 1, (M, N)).astype(np.float16)
    names = [hx.config_get(4, i)["name"] for i in range(hx.config_count(4))]
    hx.config_select(4, M, N, K, names.index(cfg_name))
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        y = hx.matmul(to_dev(x, dev), to_dev(w, dev), b_layout="nk", col_scale=to_dev(s, dev),
                      residual=to_dev(r, dev))
        torch.cuda.synchronize()
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
        hx.config_select(4, M, N, K, -1)
    assert recs and all(rc["config"] == cfg_name for rc in recs), \
        [(rc["plan"], rc["config"], rc["reason"]) for rc in recs]
    want = oracle.matmul(x, w, b_trans=True, scale_n=s.astype(np.float32), residual=r)
    assert_close(to_np(y).astype(np.float32), want.astype(np.float32), 1e-2, 2e-3, f"w8a16 split {cfg_name}")


def _quant16(x):
    """The reference's f32 pack quantisation: (x + 0) rounded to nearest even."""
    return (np.asarray(x, np.float32) + np.float32(0.0)).astype(np.float16)


@pytest.mark.parametrize("a_dt,b_dt,layout", [("f32", "f32", "kn"), ("f32", "f16", "nk"), ("f16", "f32", "kn"),
                                              ("f32", "f32", "nk")])
def test_matmul_f32_operands_quantised_at_the_pack(hx, dev, a_dt, b_dt, layout):
    """f32 operands are quantised to f16 ((x + 0), RNE) and multiplied on the
    f16 path: the result equals the oracle's product of the quantised
    operands within the f16 path's tolerance, on shapes that take the tiled
    kernel (M = 300) and the decode GEMV (M = 7)."""
    import torch
    for M in (300, 7):
        K, N = 512, 384
        a32 = rng(80 + M).normal(0, 1, (M, K)).astype(np.float32)
        b32 = rng(81 + M).normal(0, 1, (K, N) if layout == "kn" else (N, K)).astype(np.float32)
        a = a32 if a_dt == "f32" else _quant16(a32)
        b = b32 if b_dt == "f32" else _quant16(b32)
        got = to_np(hx.matmul(to_dev(a, dev), to_dev(b, dev), b_layout=layout, out_dtype=torch.float32))
        want = oracle.matmul(_quant16(a32), _quant16(b32), b_trans=(layout == "nk"), out_dtype=np.float32)
        assert_close(got, want, 1e-3, 1e-3, f"f32 operands {a_dt}.{b_dt} {layout} M={M}")


def test_f32_quantisation_special_values(hx, dev):
    """The quantisation itself, read back through an identity product (each
    value alone in its row, on the diagonal): ties round to even, values past
    65504 become infinities of their sign, and tiny values land on the f16
    subnormals or flush to zero.  (A -0 operand is not observable through a
    product: the binary32 accumulator starts at +0.)"""
    import torch
    K = 256
    vals = np.array([1.0 + 2 ** -11, 1.0 + 3 * 2 ** -11, 65504.0, 65520.0, -70000.0, 2 ** -24, 2 ** -26,
                     3 * 2 ** -25, 0.1, -1 / 3], np.float32)
    a = np.zeros((len(vals), K), np.float32)
    a[np.arange(len(vals)), np.arange(len(vals))] = vals
    eye = np.eye(K, dtype=np.float32)
    got = to_np(hx.matmul(to_dev(a, dev), to_dev(eye, dev), b_layout="kn", out_dtype=torch.float32))
    diag = got[np.arange(len(vals)), np.arange(len(vals))]
    want = _quant16(vals).astype(np.float32)
    np.testing.assert_array_equal(diag, want)
    assert diag[3] == np.inf and diag[4] == -np.inf and diag[0] == 1.0 and diag[1] == 1.0 + 4 * 2 ** -11
    assert diag[6] == 0.0 and diag[7] == 2 ** -24 * 2


def test_f32_weight_negative_zero_and_nan(hx, dev):
    """The pack's `x + 0` turns -0 into +0 (the reference's prepack contract,
    test_hmx_weight_prepack_f32.py:158-168), which the registry's byte-checked
    dedupe makes observable: an f32 weight holding -0 shares the handle of the
    f16 weight holding +0, and an f16 weight holding -0 (0x8000) gets a
    handle of its own.  A NaN weight stays a NaN (:170-194): its output
    column is NaN for every row, the other columns are the product of the
    finite weights."""
    K, N, M = 256, 512, 4
    w32 = rng(87).normal(0, 0.5, (K, N)).astype(np.float32)
    w32[::7, 3] = np.float32(-0.0)
    w32[5, ::11] = np.float32(-0.0)
    plus = _quant16(w32)
    assert not np.signbit(plus[w32 == 0]).any()
    minus = plus.copy()
    minus[5, ::11] = np.float16(-0.0)
    W = hx.ResidentWeight(to_dev(w32, dev), layout="kn")
    Wp = hx.ResidentWeight(to_dev(plus, dev), layout="kn")
    Wm = hx.ResidentWeight(to_dev(minus, dev), layout="kn")
    try:
        assert W.handle == Wp.handle and Wm.handle != W.handle
        assert W.info()["refcount"] == 2 and Wm.info()["refcount"] == 1
    finally:
        W.release(); Wp.release(); Wm.release()

    wn = w32.copy()
    nan_cols = [1, 200, 511]
    wn[17, nan_cols] = np.float32("nan")
    wn[100, 200] = -np.float32("nan")
    x = rng(88).normal(0, 1, (M, K)).astype(np.float16)
    Wn = hx.ResidentWeight(to_dev(wn, dev), layout="kn")
    try:
        got = to_np(hx.matmul_resident(to_dev(x, dev), Wn)).astype(np.float32)
    finally:
        Wn.release()
    assert np.isnan(got[:, nan_cols]).all()
    finite = np.setdiff1d(np.arange(N), nan_cols)
    assert np.isfinite(got[:, finite]).all()
    want = oracle.matmul(x, _quant16(w32)).astype(np.float32)
    assert_close(got[:, finite], want[:, finite], 1e-2, 1e-3, "finite columns of a NaN weight")


@pytest.mark.parametrize("M,N", [(8, 512), (20, 2048), (40, 512)])
def test_resident_f32_weight(hx, dev, M, N):
    """An f32 weight registers as its f16 quantisation: the resident product
    equals the argument product of the quantised weight in the same [N][K]
    orientation bit for bit (the decode GEMV, its row blocks, and the tiled
    GEMM), and an identical f16 registration shares its handle."""
    import torch
    K = 384
    w32 = rng(85).normal(0, 0.5, (K, N)).astype(np.float32)
    x = rng(86).normal(0, 1, (M, K)).astype(np.float16)
    W = hx.ResidentWeight(to_dev(w32, dev), layout="kn")
    W16 = hx.ResidentWeight(to_dev(_quant16(w32), dev), layout="kn")
    try:
        assert W.info()["dtype"] == 1 and W.handle == W16.handle and W.info()["refcount"] == 2
        got = to_np(hx.matmul_resident(to_dev(x, dev), W))
        wq = np.ascontiguousarray(_quant16(w32).T)
        ref = to_np(hx.matmul(to_dev(x, dev), to_dev(wq, dev), b_layout="nk"))
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
        want = x.astype(np.float64) @ _quant16(w32).astype(np.float64)
        assert np.abs(got.astype(np.float64) - want).max() <= 2e-3 * np.abs(want).max()
    finally:
        W.release(); W16.release()
