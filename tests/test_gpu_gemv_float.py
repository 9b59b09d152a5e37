"""GPU parity for the f16 / bf16 decode GEMV (hx_matmul and hx_matmul_resident
with M <= 16): the streaming kernel reads the K-contiguous [N][K] weight in
place (argument weights in "nk" layout, "kn" ones after the transpose into
the workspace, or the resident image).  Against the oracle's binary32
(i,k,j) product within the float-matmul tolerances (f16: rtol 1e-2 / atol
1e-3 and the reference's relative-Frobenius gate rel < 2e-3 against the f64
product; bf16: 2e-2 / 1e-2, rel < 8e-3), for every compiled configuration,
ragged N and K, the LDS-staged configs past their limit, and a column
scale.  The plan manifest shows which kernel ran."""
import numpy as np
import pytest

from conftest import assert_close, bf16_from_f32, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu

OP = {"f16": 7, "bf16": 8}
TOL = {"f16": (1e-2, 1e-3, 2e-3), "bf16": (2e-2, 1e-2, 8e-3)}


def _fp(dtype, shape, seed):
    x = rng(seed).uniform(-1.0, 1.0, shape).astype(np.float32)
    return x.astype(np.float16) if dtype == "f16" else bf16_from_f32(x)


def _vals(h, dtype):
    return oracle.bf16_bits_to_f32(h) if dtype == "bf16" else np.asarray(h, np.float32)


def _dev(h, dtype, dev):
    import torch
    t = to_dev(h.view(np.int16) if dtype == "bf16" else h, dev)
    return t.view(torch.bfloat16) if dtype == "bf16" else t


def _check(got, a, b_kn, dtype, what, scale=None):
    bf = dtype == "bf16"
    want = oracle.matmul(a, b_kn, a_bf16=bf, b_bf16=bf, out_bf16=bf,
                         scale_n=None if scale is None else scale.astype(np.float32))
    rtol, atol, gate = TOL[dtype]
    g = _vals(got, dtype)
    assert_close(g, _vals(want, dtype), rtol, atol, what)
    exact = _vals(a, dtype).astype(np.float64) @ _vals(b_kn, dtype).astype(np.float64)
    if scale is not None:
        exact = exact * scale.astype(np.float64)
    rel = np.linalg.norm(g - exact) / np.linalg.norm(exact)
    assert rel < gate, (what, rel)


def _plans(hx):
    return [r["plan"] for r in hx.manifest()["records"]]


SHAPES = [(1, 1000, 520), (3, 37, 72), (4, 4096, 4096), (5, 300, 1032), (16, 11008, 4096), (2, 100, 16384)]


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("layout", ["nk", "kn"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_decode_float_argument(hx, dev, dtype, layout, shape):
    M, N, K = shape
    a = _fp(dtype, (M, K), 40)
    b = _fp(dtype, (K, N), 41)
    bb = b if layout == "kn" else np.ascontiguousarray(b.T)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        c = hx.matmul(_dev(a, dtype, dev), _dev(bb, dtype, dev), b_layout=layout)
        plans = _plans(hx)
    finally:
        hx.manifest_enable(False)
    # [K][N] weights stream in place when N % 8 == 0, else after the
    # transpose; one row against an [N][K] weight (K <= 8192): whole rows
    # per wave
    want = ("gemv-kn" if layout == "kn" and N % 8 == 0 else
            "gemv-rowdot" if layout == "nk" and M == 1 and K <= 8192 else "gemv-stream")
    assert plans == [want], plans
    _check(to_np(c), a, b, dtype, f"decode {dtype} {layout} {shape}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(1, 8192, 8192), (3, 4096, 1032), (16, 128, 4096), (1, 136, 24), (7, 11008, 256)],
                         ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("scale", [None, "f16", "f32"])
def test_decode_kn_in_place(hx, dev, dtype, shape, scale):
    """[K][N] weights read in place (no transpose): one K part or several
    with the binary32 partial merge, with an f16 or f32 column scale, and a
    row stride wider than N."""
    import torch
    M, N, K = shape
    a = _fp(dtype, (M, K), 100)
    b = _fp(dtype, (K, N), 101)
    s = None if scale is None else rng(102).uniform(0.5, 1.5, N).astype(np.float16)
    wide = _dev(np.zeros((K, N + 24), b.dtype), dtype, dev)
    wide[:, :N] = _dev(b, dtype, dev)
    sd = None if s is None else (to_dev(s, dev) if scale == "f16" else to_dev(s.astype(np.float32), dev))
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        c = hx.matmul(_dev(a, dtype, dev), wide[:, :N], b_layout="kn", col_scale=sd)
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    assert [(r["plan"], r["weight"]) for r in recs] == [("gemv-kn", "argument-kn")], recs
    torch.cuda.synchronize()
    _check(to_np(c), a, b, dtype, f"kn {dtype} {shape} {scale}", scale=s)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(1, 1000, 4160), (4, 300, 8192), (7, 37, 144), (16, 523, 1024)],
                         ids=lambda s: "x".join(map(str, s)))
def test_decode_float_resident_every_config(hx, dev, dtype, shape):
    """Every config of the decode family on the resident image (LDS-staged
    configs run as their base configs past M = 4 or their LDS limit), each
    deterministic, with a per-column scale."""
    M, N, K = shape
    a = _fp(dtype, (M, K), 50)
    b = _fp(dtype, (K, N), 51)
    s = rng(52).uniform(0.5, 1.5, N).astype(np.float16)
    rw = hx.ResidentWeight(_dev(b, dtype, dev), to_dev(s, dev), layout="kn")
    ad = _dev(a, dtype, dev)
    op = OP[dtype]
    try:
        n = hx.config_count(op)
        assert n == hx.config_count(6)
        for cfg in range(n):
            hx.config_select(op, M, N, K, cfg)
            try:
                got = to_np(hx.matmul_resident(ad, rw))
                again = to_np(hx.matmul_resident(ad, rw))
            finally:
                hx.config_select(op, M, N, K, -1)
            _check(got, a, b, dtype, f"resident {dtype} {shape} cfg {cfg}", scale=s)
            assert np.array_equal(got.view(np.uint16), again.view(np.uint16)), f"cfg {cfg}: not deterministic"
    finally:
        rw.release()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_decode_float_tuner_shape(hx, dev, dtype):
    """The reference tuner's decode shape (1, 8192, 8192): a registered
    weight runs the decode GEMV on its packed image, an argument [N][K]
    weight the row-dot kernel (whole rows per wave); both match the oracle
    and repeat bit for bit."""
    M, N, K = 1, 8192, 8192
    a = _fp(dtype, (M, K), 60)
    b = _fp(dtype, (K, N), 61)
    bt = _dev(np.ascontiguousarray(b.T), dtype, dev)
    ad = _dev(a, dtype, dev)
    rw = hx.ResidentWeight(bt, None, layout="nk")
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        res = to_np(hx.matmul_resident(ad, rw))
        arg = to_np(hx.matmul(ad, bt, b_layout="nk"))
        plans = [r["plan"] for r in hx.manifest()["records"]]
        res2 = to_np(hx.matmul_resident(ad, rw))
        arg2 = to_np(hx.matmul(ad, bt, b_layout="nk"))
    finally:
        hx.manifest_enable(False)
        rw.release()
    assert plans == ["gemv-packed", "gemv-rowdot"], plans
    assert np.array_equal(res.view(np.uint16), res2.view(np.uint16))
    assert np.array_equal(arg.view(np.uint16), arg2.view(np.uint16))
    _check(res, a, b, dtype, f"tuner shape resident {dtype}")
    _check(arg, a, b, dtype, f"tuner shape argument {dtype}")


def test_decode_float_falls_back_off_grid(hx, dev):
    """K not a multiple of 8 is refused by the streaming kernel; the call
    still runs (the generic MFMA GEMM) and matches the oracle."""
    M, N, K = 2, 64, 100
    a = _fp("f16", (M, K), 70)
    b = _fp("f16", (K, N), 71)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        c = hx.matmul(to_dev(a, dev), to_dev(b, dev), b_layout="kn")
        plans = _plans(hx)
    finally:
        hx.manifest_enable(False)
    assert "gemv-stream" not in plans, plans
    _check(to_np(c), a, b, "f16", "off-grid decode")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("layout", ["kn", "nk"])
@pytest.mark.parametrize("mk", [(8192, 4096), (300, 520), (17, 64), (40, 9000)], ids=lambda s: "x".join(map(str, s)))
def test_matvec_n_is_one(hx, dev, dtype, layout, mk):
    """N = 1 (the reference tuner's (M, K, 1) rows): A's rows are dotted
    with b, whole rows per wave (K <= 8192), or A is streamed as the decode
    GEMV's weight with b as the single activation row."""
    M, K = mk
    a = _fp(dtype, (M, K), 80)
    b = _fp(dtype, (K, 1), 81)
    bb = b if layout == "kn" else np.ascontiguousarray(b.T)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        c = hx.matmul(_dev(a, dtype, dev), _dev(bb, dtype, dev), b_layout=layout)
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    plan = "gemv-rowdot" if K <= 8192 else "gemv-stream"
    assert [(r["plan"], r["weight"], r["reason"]) for r in recs] == [(plan, "swapped-a-streamed", "n-is-one")]
    _check(to_np(c), a, b, dtype, f"matvec {dtype} {layout} {mk}")


def test_matvec_n_is_one_fallbacks(hx, dev):
    """A column scale, or an output column that is not contiguous, keeps the
    N = 1 product on the GEMM path; the result is unchanged."""
    import torch
    M, K = 256, 512
    a = _fp("f16", (M, K), 90)
    b = _fp("f16", (K, 1), 91)
    s = rng(92).uniform(0.5, 1.5, 1).astype(np.float16)
    out = torch.zeros((M, 2), dtype=torch.float16, device=dev)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        c1 = hx.matmul(to_dev(a, dev), to_dev(b, dev), col_scale=to_dev(s, dev))
        hx.matmul(to_dev(a, dev), to_dev(b, dev), out=out[:, :1])
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    assert all(r["plan"] != "gemv-stream" for r in recs), recs
    _check(to_np(c1), a, b, "f16", "matvec scaled", scale=s)
    _check(to_np(out[:, :1].contiguous()), a, b, "f16", "matvec strided out")
    assert not to_np(out[:, 1:].contiguous()).any()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(17, 2048, 520), (24, 4096, 4096), (20, 11008, 1024), (23, 2053, 72),
                                   (32, 4096, 1024), (17, 1000, 520), (33, 4096, 4096), (48, 11008, 1024),
                                   (64, 300, 8192), (63, 37, 72), (48, 11008, 4096), (64, 4096, 11008)],
                         ids=lambda s: "x".join(map(str, s)))
def test_decode_float_row_blocks(hx, dev, dtype, shape):
    """16 < M <= 32 with N >= 2048: the streaming kernel with 2 blocks of 16
    activation rows (each weight fragment feeds every block), on a registered
    weight's packed image, and on an argument [N][K] weight read in place up
    to N = 4096; on the packed image also 32 < M <= 64 with four blocks at
    641..768 column tiles and K >= 4096; fewer columns or more rows: the
    tiled GEMM.  Same numerics either way."""
    M, N, K = shape
    rows = 16 < M <= 32 and 2048 <= N <= 4096
    rows_resident = (16 < M <= 32 and N >= 2048) or (32 < M <= 64 and 641 <= -(-N // 16) <= 768 and K >= 4096)
    a = _fp(dtype, (M, K), 110)
    b = _fp(dtype, (K, N), 111)
    bt = _dev(np.ascontiguousarray(b.T), dtype, dev)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        c = hx.matmul(_dev(a, dtype, dev), bt, b_layout="nk")
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    if rows:
        assert [r["plan"] for r in recs] == ["gemv-stream"] and recs[0]["config"].startswith("rows"), recs
    else:
        assert [r["plan"] for r in recs] in (["mfma-tiled"], ["mfma-generic"]), recs  # N = 37: generic
    _check(to_np(c), a, b, dtype, f"rows {dtype} {shape}")
    rw = hx.ResidentWeight(bt, None, layout="nk")
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        got = to_np(hx.matmul_resident(_dev(a, dtype, dev), rw))
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
        rw.release()
    if rows_resident:
        assert [(r["plan"], r["weight"]) for r in recs] == [("gemv-packed", "resident-packed")], recs
        assert recs[0]["config"].startswith("rows"), recs
    else:
        assert [r["plan"] for r in recs] in (["mfma-tiled"], ["mfma-generic"]), recs
    _check(got, a, b, dtype, f"rows resident {dtype} {shape}")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(3, 523, 1064), (16, 700, 264), (20, 2053, 264)],
                         ids=lambda s: "x".join(map(str, s)))
def test_packed_image_matches_in_place(hx, dev, dtype, shape):
    """A registered f16 / bf16 weight's packed image holds, in every lane of
    every wave load, the same 16 bytes the in-place read of the [N][K] weight
    gives that lane: under every config of the family the resident product
    equals the argument product bit for bit (ragged N, K not a multiple of
    the 32-deep chunk)."""
    M, N, K = shape
    a = _fp(dtype, (M, K), 130)
    bt = _fp(dtype, (N, K), 131)
    ad, bd = _dev(a, dtype, dev), _dev(bt, dtype, dev)
    rw = hx.ResidentWeight(bd, None, layout="nk")
    op = OP[dtype]
    try:
        for cfg in range(hx.config_count(op)):
            hx.config_select(op, M, N, K, cfg)
            try:
                got = to_np(hx.matmul_resident(ad, rw))
                ref = to_np(hx.matmul(ad, bd, b_layout="nk"))
            finally:
                hx.config_select(op, M, N, K, -1)
            assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), f"cfg {cfg}"
        _check(got, a, np.ascontiguousarray(bt.T), dtype, f"packed {dtype} {shape}")
    finally:
        rw.release()


def test_decode_row_blocks_every_config(hx, dev):
    """Every config of the shared table at M = 24 (f16, N = 2059; int8,
    N = 523): configs with too few row blocks run as the row-block default."""
    M, N, K = 24, 2059, 1024
    a = _fp("f16", (M, K), 120)
    b = _fp("f16", (K, N), 121)
    rw = hx.ResidentWeight(_dev(b, "f16", dev), None, layout="kn")
    ad = _dev(a, "f16", dev)
    try:
        for cfg in range(hx.config_count(7)):
            hx.config_select(7, M, N, K, cfg)
            try:
                got = to_np(hx.matmul_resident(ad, rw))
            finally:
                hx.config_select(7, M, N, K, -1)
            _check(got, a, b, "f16", f"rows every config {cfg}")
    finally:
        rw.release()
    M, N = 24, 523
    x = rng(122).normal(0, 1, (M, K)).astype(np.float16)
    w = rng(123).integers(-127, 128, (K, N), dtype=np.int8)
    s = rng(124).uniform(0.001, 0.02, N).astype(np.float16)
    want = oracle.matmul(x, w, scale_n=s.astype(np.float32)).astype(np.float32)
    rw = hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev))
    xd = to_dev(x, dev)
    try:
        for cfg in range(hx.config_count(6)):
            hx.config_select(6, M, N, K, cfg)
            try:
                got = to_np(hx.matmul_resident(xd, rw)).astype(np.float32)
            finally:
                hx.config_select(6, M, N, K, -1)
            assert_close(got, want, 1e-2, 1e-3, f"int8 rows cfg {cfg}")
    finally:
        rw.release()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
@pytest.mark.parametrize("shape", [(16, 4096, 11008), (9, 523, 4104)], ids=lambda s: "x".join(map(str, s)))
def test_decode_float_split_k(hx, dev, dtype, shape):
    """The K split over workgroups on f16 / bf16 weights, on the packed image
    and read in place (an argument [N][K] weight), every split config:
    within the oracle's tolerances and repeatable bit for bit."""
    import torch
    M, N, K = shape
    a = _fp(dtype, (M, K), 60)
    b = _fp(dtype, (K, N), 61)
    bnk = np.ascontiguousarray(b.T)
    op = OP[dtype]
    rw = hx.ResidentWeight(_dev(b, dtype, dev), layout="kn")
    ad, bd = _dev(a, dtype, dev), _dev(bnk, dtype, dev)
    splits = [i for i in range(hx.config_count(op)) if hx.config_get(op, i)["split_k"] > 1]
    assert len(splits) == 9
    try:
        for cfg in splits:
            hx.config_select(op, M, N, K, cfg)
            try:
                res = [to_np(hx.matmul_resident(ad, rw)) for _ in range(2)]
                arg = [to_np(hx.matmul(ad, bd, b_layout="nk")) for _ in range(2)]
            finally:
                hx.config_select(op, M, N, K, -1)
            for got, what in ((res, "packed"), (arg, "in place")):
                _check(got[0], a, b, dtype, f"{what} {dtype} {shape} cfg {cfg}")
                assert np.array_equal(got[0].view(np.uint16), got[1].view(np.uint16)), f"{what} cfg {cfg}"
    finally:
        rw.release()
