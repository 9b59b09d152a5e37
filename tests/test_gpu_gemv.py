"""GPU parity for the W8A16 decode GEMV (M in {1, 4, 16},
N = 11008, K = 4096, int8 weights, per-output-channel fp16 scales, fp16
activations N(0,1), binary32 accumulation, fp16 out) within rtol 1e-2 /
atol 1e-3 of the oracle, for every compiled configuration, both weight
orientations, ragged N / K, and the resident-weight path."""
import numpy as np
import pytest

from conftest import assert_close, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu


def case(M, N, K, seed=0):
    x = rng(seed).normal(0, 1, (M, K)).astype(np.float16)
    w = rng(seed + 1).integers(-127, 128, (K, N), dtype=np.int8)
    s = rng(seed + 2).uniform(0.001, 0.02, N).astype(np.float16)
    return x, w, s


@pytest.fixture(scope="module")
def c3():
    N, K = 11008, 4096
    x, w, s = case(16, N, K, seed=100)
    wt = np.ascontiguousarray(w.T)
    want = {M: oracle.matmul(np.ascontiguousarray(x[:M]), wt, b_trans=True, scale_n=s.astype(np.float32))
            for M in (1, 4, 16)}
    return x, w, wt, s, want


@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_c3_kn(hx, dev, c3, M):
    x, w, wt, s, want = c3
    y = hx.gemv_w8a16(to_dev(np.ascontiguousarray(x[:M]), dev), to_dev(w, dev), to_dev(s, dev), w_layout="kn")
    assert_close(to_np(y).astype(np.float32), want[M].astype(np.float32), 1e-2, 1e-3, f"gemv M={M}")


@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_c3_every_config(hx, dev, c3, M):
    """Every compiled decode-GEMV configuration (the resident, fragment-packed
    path the autotuner searches) is within tolerance and deterministic."""
    x, w, wt, s, want = c3
    N, K = wt.shape
    xt = to_dev(np.ascontiguousarray(x[:M]), dev)
    rw = hx.ResidentWeight(to_dev(wt, dev), to_dev(s, dev), layout="nk")
    try:
        for cfg in range(hx.config_count(6)):
            hx.config_select(6, M, N, K, cfg)
            try:
                got = to_np(hx.matmul_resident(xt, rw))
                again = to_np(hx.matmul_resident(xt, rw))
            finally:
                hx.config_select(6, M, N, K, -1)
            assert_close(got.astype(np.float32), want[M].astype(np.float32), 1e-2, 1e-3, f"cfg {cfg} M={M}")
            assert np.array_equal(got.view(np.uint16), again.view(np.uint16)), f"cfg {cfg}: not deterministic"
    finally:
        rw.release()


@pytest.mark.parametrize("shape", [(3, 1000, 4096), (16, 11008, 4112), (7, 37, 144), (2, 5000, 16)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemv_ragged(hx, dev, shape):
    M, N, K = shape
    x, w, s = case(M, N, K, seed=200)
    y = hx.gemv_w8a16(to_dev(x, dev), to_dev(w, dev), to_dev(s, dev))
    want = oracle.matmul(x, w, scale_n=s.astype(np.float32))
    assert_close(to_np(y).astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, f"ragged {shape}")


def test_gemv_resident_matches_raw(hx, dev, c3):
    """The resident (registered, fragment-packed) weight and the raw call agree
    within tolerance (they sum in different orders), and registering identical
    content returns the same handle."""
    x, w, wt, s, want = c3
    wd, sd = to_dev(w, dev), to_dev(s, dev)
    rw = hx.ResidentWeight(wd, sd, layout="kn")
    rw2 = hx.ResidentWeight(to_dev(wt, dev), sd, layout="nk")
    try:
        assert rw.handle == rw2.handle, "identical content must map to one resident image"
        assert rw.info()["refcount"] == 2
        for M in (1, 4, 16):
            xm = to_dev(np.ascontiguousarray(x[:M]), dev)
            y_res = to_np(hx.matmul_resident(xm, rw))
            y_raw = to_np(hx.gemv_w8a16(xm, wd, sd))
            assert_close(y_res.astype(np.float32), y_raw.astype(np.float32), 1e-2, 1e-3, "resident vs raw")
            assert_close(y_res.astype(np.float32), want[M].astype(np.float32), 1e-2, 1e-3, "resident")
    finally:
        rw2.release()
        rw.release()


@pytest.mark.parametrize("shape", [(5, 1000, 4160), (16, 37, 200), (1, 11008, 64), (3, 20, 8),
                                   (4, 300, 8192), (2, 100, 16384)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemv_resident_ragged(hx, dev, shape):
    """Packed decode path with N not a multiple of 16 and K not a multiple of
    64 (the image is zero-padded; K % 8 == 0 is required for this path), and
    every config including the LDS-staged ones past their LDS limit (M = 4,
    K = 8192 and M = 2, K = 16384 run as their base configs)."""
    M, N, K = shape
    x, w, s = case(M, N, K, seed=300)
    rw = hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev))
    want = oracle.matmul(x, w, scale_n=s.astype(np.float32))
    xd = to_dev(x, dev)
    try:
        for cfg in range(hx.config_count(6)):
            hx.config_select(6, M, N, K, cfg)
            try:
                y = to_np(hx.matmul_resident(xd, rw))
            finally:
                hx.config_select(6, M, N, K, -1)
            assert_close(y.astype(np.float32), want.astype(np.float32), 1e-2, 1e-3,
                         f"packed ragged {shape} cfg {cfg}")
    finally:
        rw.release()


@pytest.mark.parametrize("shape", [(1, 11008, 4096), (4, 4096, 1032), (16, 256, 8192), (2, 16, 24)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemv_kn_in_place(hx, dev, shape):
    """int8 weights in the linalg [K][N] orientation are streamed in place
    (no transpose): bytes transposed and widened in registers, one K part or
    several with the binary32 partial merge; a row stride wider than N."""
    import torch
    M, N, K = shape
    x, w, s = case(M, N, K, seed=400)
    wide = torch.zeros((K, N + 32), dtype=torch.int8, device=dev)
    wide[:, :N] = to_dev(w, dev)
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        y = hx.gemv_w8a16(to_dev(x, dev), wide[:, :N], to_dev(s, dev), w_layout="kn")
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    assert [(r["plan"], r["weight"], r["b"]) for r in recs] == [("gemv-kn", "argument-kn", "i8")], recs
    want = oracle.matmul(x, w, scale_n=s.astype(np.float32))
    assert_close(to_np(y).astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, f"kn in place {shape}")


@pytest.mark.parametrize("shape,scale32", [((11008, 4096), False), ((37, 1040), True), ((100, 8192), False),
                                           ((100, 520), False), ((64, 8208), True)],
                         ids=["11008x4096", "37x1040-f32scale", "100x8192", "100x520", "64x8208"])
def test_gemv_one_row_nk(hx, dev, shape, scale32):
    """One activation row against an [N][K] int8 argument weight: whole rows
    per wave (K % 16 == 0 and K <= 8192), else the streaming GEMV; f16 or f32
    scale, ragged N, against the oracle."""
    N, K = shape
    x, w, s = case(1, N, K, seed=N + K)
    wt = np.ascontiguousarray(w.T)
    sc = s.astype(np.float32) if scale32 else s
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        y = hx.gemv_w8a16(to_dev(x, dev), to_dev(wt, dev), to_dev(sc, dev), w_layout="nk")
        plans = [r["plan"] for r in hx.manifest()["records"]]
    finally:
        hx.manifest_enable(False)
    assert plans == ["gemv-rowdot" if (K % 16 == 0 and K <= 8192) else plans[0]], plans
    if not (K % 16 == 0 and K <= 8192):
        assert plans[0] != "gemv-rowdot", plans
    want = oracle.matmul(x, wt, b_trans=True, scale_n=s.astype(np.float32))
    assert_close(to_np(y).astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, f"one row {shape}")


def _split_configs(hx):
    return [(i, hx.config_get(6, i)) for i in range(hx.config_count(6)) if hx.config_get(6, i)["split_k"] > 1]


@pytest.mark.parametrize("shape", [(16, 4096, 11008), (9, 1000, 4112), (12, 37, 640), (6, 300, 8200),
                                   (24, 4096, 11008), (31, 300, 8200), (40, 4096, 11008), (64, 300, 8200)],
                         ids=lambda s: "x".join(map(str, s)))
def test_gemv_split_k_over_workgroups(hx, dev, shape):
    """Configs that split K over workgroups (M > 4; up to 16 rows per row
    block: 32 for two blocks, 64 for four; a config whose blocks cannot hold
    M runs the row-block default): every part's binary32 partials and the last
    workgroup's sum in part order.  Within tolerance of
    the oracle, bit-identical over repeated calls (the parts are added in
    the same order whichever workgroup finishes last, and every call returns
    the counters to zero for the next), with N not a multiple of the tile
    group and K not a multiple of the parts."""
    M, N, K = shape
    x, w, s = case(M, N, K, seed=700)
    rw = hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev))
    want = oracle.matmul(x, w, scale_n=s.astype(np.float32)).astype(np.float32)
    xd = to_dev(x, dev)
    splits = _split_configs(hx)
    assert {c["split_k"] for _, c in splits} == {2, 4}, splits
    try:
        for cfg, info in splits:
            hx.config_select(6, M, N, K, cfg)
            try:
                runs = [to_np(hx.matmul_resident(xd, rw)) for _ in range(3)]
            finally:
                hx.config_select(6, M, N, K, -1)
            assert_close(runs[0].astype(np.float32), want, 1e-2, 1e-3, f"{info['name']} {shape}")
            for r in runs[1:]:
                assert np.array_equal(r.view(np.uint16), runs[0].view(np.uint16)), f"{info['name']}: not repeatable"
    finally:
        rw.release()


def test_gemv_split_k_few_rows_run_the_base(hx, dev):
    """With M <= 4 a split config runs its base config (the few-row
    reduction finishes in place): bit-identical to the base pinned itself,
    and the tuner refuses it with a reason."""
    M, N, K = 4, 4096, 11008
    x, w, s = case(M, N, K, seed=710)
    rw = hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev))
    xd = to_dev(x, dev)
    names = [hx.config_get(6, i)["name"] for i in range(hx.config_count(6))]
    base = {"gemv_packed_ct2_kw16_s2": "gemv_packed_ct2_kw8", "gemv_packed_ct4_kw16_s4": "gemv_packed_ct4_kw16",
            "gemv_packed_ct6_kw16_s2": "gemv_packed_ct3_kw16", "gemv_packed_ct1_kw16_s2": "gemv_packed_ct1_kw16",
            "gemv_packed_ct2_kw16_s4": "gemv_packed_ct2_kw8", "gemv_packed_ct4_kw16_s4_e": "gemv_packed_ct4_kw16",
            "gemv_rows2_ct4_kw16_s4_e": "gemv_packed_ct4_kw16", "gemv_rows2_ct2_kw16_s2_e": "gemv_packed_ct2_kw8",
            "gemv_rows4_ct4_kw8_s4_e": "gemv_rows4_ct4_kw8"}
    try:
        for sname, bname in base.items():
            got = []
            for name in (sname, bname):
                hx.config_select(6, M, N, K, names.index(name))
                try:
                    got.append(to_np(hx.matmul_resident(xd, rw)))
                finally:
                    hx.config_select(6, M, N, K, -1)
            assert np.array_equal(got[0].view(np.uint16), got[1].view(np.uint16)), sname
    finally:
        rw.release()
    r = hx.search.tune(6, M, N, K, canary_reference_us=-1.0, reps=3, budget_us=20_000.0, min_iters=5,
                       max_iters=40, pin=False)
    reasons = {e["cfg"]: e.get("reason") for e in r["entries"]}
    assert all(reasons[n] == "split-rows" for n in base), reasons


def test_gemv_split_k_is_the_default_where_it_pays(hx, dev):
    """The untuned choice: 12 rows or more on at most 256 tiles with K of
    8192 or more split K over workgroups (int8: four tiles, four parts),
    and 5 to 12 rows on at most 128 tiles (one tile, two parts); 8 rows on
    256 tiles, or N = 11008 (688 tiles), do not."""
    N, K = 4096, 11008
    x, w, s = case(16, N, K, seed=720)
    rw = hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev))
    x2, w2, s2 = case(16, 11008, 4096, seed=721)
    rw2 = hx.ResidentWeight(to_dev(w2, dev), to_dev(s2, dev))
    x3, w3, s3 = case(8, 2048, 8192, seed=722)
    rw3 = hx.ResidentWeight(to_dev(w3, dev), to_dev(s3, dev))
    hx.manifest_clear()
    prev = hx.manifest_enable(True)
    try:
        for M in (16, 8):
            hx.matmul_resident(to_dev(np.ascontiguousarray(x[:M]), dev), rw)
        hx.matmul_resident(to_dev(x2, dev), rw2)
        hx.matmul_resident(to_dev(x3, dev), rw3)
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(prev)
        rw.release(); rw2.release(); rw3.release()
    got = {(r["m"], r["n"]): r["config"] for r in recs}
    assert got[(16, 4096)] == "packed_ct4_kw16_s4_e", got
    assert "_s" not in got[(8, 4096)][-3:] and "_s" not in got[(16, 11008)][-3:], got
    # at most 128 tiles (N = 2048), K = 8192: one tile per workgroup over two parts
    assert got[(8, 2048)] == "packed_ct1_kw16_s2", got


def test_gemv_defaults_follow_the_ab(hx):
    """The untuned defaults at the C3 shapes, the FFN's down projection and
    the reference tuner's fp16 decode shapes are the configs that the
    interleaved A/B in one process (bench.py --gemv-ab and the f16 decode
    sweep) timed fastest: three tiles over 16 waves with every slice load
    issued ahead at N = 11008; the four-part K split at 16 rows of the down
    projection and one tile over 8 waves at 8; for an f16 packed image with
    one row, 16 waves at 8192 x 8192 and 8 at 4096 x 16384, and on the down
    projection's shape four parts from 13 rows, two up to 12; past 16 rows
    two row blocks, split over K on the down projection's shape; past 32
    rows four row blocks, three tiles over 16 waves at N = 11008 and four
    tiles over four K parts on the down projection's shape."""
    want = {(6, 1, 11008, 4096): "packed_ct3_kw16_e", (6, 4, 11008, 4096): "packed_ct3_kw16_e",
            (6, 16, 11008, 4096): "packed_ct3_kw16_e", (6, 16, 4096, 11008): "packed_ct4_kw16_s4_e",
            (6, 8, 4096, 11008): "packed_ct1_kw8_e", (7, 1, 8192, 8192): "packed_ct1_kw16_xl",
            (7, 1, 4096, 16384): "packed_ct1_kw8_xl", (7, 16, 4096, 11008): "packed_ct4_kw16_s4_e",
            (7, 12, 4096, 11008): "packed_ct2_kw16_s2", (7, 8, 4096, 4096): "packed_ct1_kw8_e",
            (6, 17, 4096, 11008): "rows2_ct2_kw16_s2_e", (6, 24, 4096, 11008): "rows2_ct4_kw16_s4_e",
            (6, 24, 11008, 4096): "rows2_ct3_kw8", (6, 33, 11008, 4096): "rows4_ct3_kw16_e",
            (6, 48, 11008, 4096): "rows4_ct3_kw16_e", (6, 33, 4096, 11008): "rows4_ct4_kw8_s4_e",
            (6, 64, 4096, 11008): "rows4_ct4_kw8_s4_e"}
    got = {k: hx.config_get(k[0], hx.config_lookup(*k))["name"] for k in want}
    assert all(got[k].endswith(v) for k, v in want.items()), got


def test_gemv_four_row_blocks_route(hx, dev):
    """A registered int8 weight takes the packed GEMV's four row blocks past
    32 rows only where they beat the tiled GEMM: on the down projection's
    shape (4096 x 11008) up to 64 rows, at N = 11008, K = 4096 up to 48;
    65 rows, 64 rows at N = 11008, and a narrow weight take the GEMM.  Each
    result is within the oracle's tolerance."""
    cases = [(40, 4096, 11008, "gemv"), (64, 4096, 11008, "gemv"), (65, 4096, 11008, "tiled"),
             (48, 11008, 4096, "gemv"), (64, 11008, 4096, "tiled"), (40, 512, 512, "tiled")]
    for M, N, K, route in cases:
        x, w, s = case(M, N, K, seed=760 + M)
        rw = hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev))
        hx.manifest_clear()
        hx.manifest_enable(True)
        try:
            y = hx.matmul_resident(to_dev(x, dev), rw)
            plans = [r["plan"] for r in hx.manifest()["records"]]
        finally:
            hx.manifest_enable(False)
            rw.release()
        if route == "gemv":
            assert plans and all(p.startswith("gemv") for p in plans), (M, N, K, plans)
        else:
            assert plans and all(p.startswith("mfma") for p in plans), (M, N, K, plans)
        want = oracle.matmul(x, w, scale_n=s.astype(np.float32)).astype(np.float32)
        assert_close(to_np(y).astype(np.float32), want, 1e-2, 1e-3, f"{M}x{N}x{K}")


@pytest.mark.parametrize("M", [1, 4, 16])
def test_gemv_load_schedule_keeps_the_bits(hx, dev, M):
    """The `_e` configs change only when the slice's loads issue: each one
    gives the bits of its twin with the compiler's load schedule (same
    tiles, waves, K split and summation order), on the int8 image at the C3
    width and on an f16 image."""
    import torch
    twins = {"gemv_packed_ct3_kw16_e": "gemv_packed_ct3_kw16", "gemv_packed_ct1_kw8_e": "gemv_packed_ct1_kw8",
             "gemv_packed_ct1_kw16_e": "gemv_packed_ct1_kw16",
             "gemv_packed_ct4_kw16_s4_e": "gemv_packed_ct4_kw16_s4"}
    N, K = 11008, 4096
    x, w, s = case(M, N, K, seed=730 + M)
    g = torch.Generator(device=dev).manual_seed(731 + M)
    wf = torch.empty((N, K), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
    xf = torch.randn((M, K), dtype=torch.float16, device=dev, generator=g)
    for op, rw, xd in ((6, hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev)), to_dev(x, dev)),
                       (7, hx.ResidentWeight(wf, None, layout="nk"), xf)):
        names = [hx.config_get(op, i)["name"] for i in range(hx.config_count(op))]
        try:
            for e, base in twins.items():
                got = []
                for name in (e, base):
                    hx.config_select(op, M, N, K, names.index(name))
                    try:
                        got.append(to_np(hx.matmul_resident(xd, rw)))
                    finally:
                        hx.config_select(op, M, N, K, -1)
                assert np.array_equal(got[0].view(np.uint16), got[1].view(np.uint16)), f"op {op} {e} M={M}"
        finally:
            rw.release()
