"""GPU parity for the persistent GEMM configs, the K split merged inside the
kernel, and the clock probe.

* Persistent configs (one workgroup per CU walking consecutive M-tiles of a
  B strip, each tile's epilogue overlapping the next tile's first K stages)
  run the same K loop as the one-tile-per-workgroup config of the same tile
  and stage width, so their outputs must equal that config's bit for bit --
  and, for int8, the oracle's.  Shapes give one, two and an uneven number
  of tiles per workgroup; shapes with edge tiles and 32-bit outputs run the
  one-tile kernel instead, also checked.
* The K split merges inside the kernel: the last part of each tile adds the
  parts' binary32 partials in part order from zero, then scales and rounds.
  Each part's partial is what the unsplit kernel computes over that part's
  K range (same tile, same stages, same order), so the split output must
  equal RNE(((0 + P0) + P1) * s) computed on the host from those partials,
  bit for bit.
* The clock probe counts one stamp per workgroup and reads a plausible
  shader clock.
"""
import numpy as np
import pytest

from conftest import rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu

GEMM_I8, MATMUL_F16, MATMUL_W8, SWIGLU_W8 = 1, 2, 4, 5


def names_of(hx, op):
    return [hx.config_get(op, i)["name"] for i in range(hx.config_count(op))]


def pinned(hx, op, shape, name):
    """Context manager pinning config `name` of family `op` at `shape`."""
    import contextlib

    @contextlib.contextmanager
    def cm():
        idx = names_of(hx, op).index(name)
        hx.config_select(op, *shape, idx)
        try:
            yield
        finally:
            hx.config_select(op, *shape, -1)
    return cm()


def i8(shape, seed):
    return rng(seed).integers(-127, 128, shape, dtype=np.int8)


# (M, N, K): 256x256 tiles -> 256 (one per CU), 306 (one or two), 576 (two
# or three) tiles; 128x256 tiles -> twice as many
I8_SHAPES = [(4096, 4096, 256), (4352, 4608, 192), (4608, 8192, 128)]


@pytest.mark.parametrize("shape", I8_SHAPES, ids=lambda s: "x".join(map(str, s)))
@pytest.mark.parametrize("name,base", [("256x256_w2x4_bk64_p", "256x256_w2x4_bk64"),
                                       ("128x256_w2x4_p", None)])
def test_i8_persistent_exact(hx, dev, shape, name, base):
    """int8 persistent configs: fp16 and bf16 dequant outputs (the
    persistent kernel) bit-exact against the oracle, int32 output (the
    one-tile kernel) exact, and equal to the base config's output."""
    import torch
    M, N, K = shape
    a, bt = i8((M, K), 900 + M), i8((N, K), 901 + N)
    sa = rng(902).uniform(0.001, 0.02, M).astype(np.float32)
    sb = rng(903).uniform(0.001, 0.02, N).astype(np.float32)
    acc = oracle.gemm_i8_i32(a, bt, b_trans=True)
    ad, bd, sad, sbd = to_dev(a, dev), to_dev(bt, dev), to_dev(sa, dev), to_dev(sb, dev)
    hx.manifest_clear()
    hx.manifest_enable(True)
    try:
        with pinned(hx, GEMM_I8, shape, name):
            c16 = to_np(hx.gemm_i8(ad, bd, b_layout="nk", row_scale=sad, col_scale=sbd, out_dtype=torch.float16))
            cb = to_np(hx.gemm_i8(ad, bd, b_layout="nk", row_scale=sad, col_scale=sbd, out_dtype=torch.bfloat16))
            c32 = to_np(hx.gemm_i8(ad, bd, b_layout="nk"))
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
    assert {r["config"] for r in recs} == {name}, recs
    want16 = oracle.dequant_i32_f16(acc, sa, sb)
    assert np.array_equal(c16.view(np.uint16), want16.view(np.uint16))
    v32 = (acc.astype(np.float32) * sa[:, None]) * sb[None, :]
    assert np.array_equal(cb, oracle.f32_to_bf16_bits(v32))
    assert np.array_equal(c32, acc)
    if base:
        with pinned(hx, GEMM_I8, shape, base):
            b16 = to_np(hx.gemm_i8(ad, bd, b_layout="nk", row_scale=sad, col_scale=sbd, out_dtype=torch.float16))
        assert np.array_equal(b16.view(np.uint16), c16.view(np.uint16))


def test_i8_persistent_edge_shape_runs_one_tile_kernel(hx, dev):
    """Edge tiles: the persistent config runs the one-tile kernel, exact."""
    import torch
    M, N, K = 1000, 776, 320
    a, bt = i8((M, K), 910), i8((N, K), 911)
    sa = rng(912).uniform(0.001, 0.02, M).astype(np.float32)
    sb = rng(913).uniform(0.001, 0.02, N).astype(np.float32)
    acc = oracle.gemm_i8_i32(a, bt, b_trans=True)
    for name in ("256x256_w2x4_bk64_p", "128x256_w2x4_p"):
        with pinned(hx, GEMM_I8, (M, N, K), name):
            c16 = to_np(hx.gemm_i8(to_dev(a, dev), to_dev(bt, dev), b_layout="nk", row_scale=to_dev(sa, dev),
                                   col_scale=to_dev(sb, dev), out_dtype=torch.float16))
        assert np.array_equal(c16.view(np.uint16), oracle.dequant_i32_f16(acc, sa, sb).view(np.uint16)), name


@pytest.mark.parametrize("shape", [(4096, 4608, 512), (4096, 4096, 384)], ids=lambda s: "x".join(map(str, s)))
def test_w8_persistent_equals_one_tile(hx, dev, shape):
    """W8A16 (f16 activations, int8 weights widened in registers, column
    scales): the persistent 256x256 config equals the one-tile 256x256
    config bit for bit (same K loop), and both are within the float gates
    of the oracle."""
    import torch
    M, N, K = shape
    x = rng(920).normal(0, 1, (M, K)).astype(np.float16)
    w = i8((N, K), 921)
    s = rng(922).uniform(0.001, 0.02, N).astype(np.float16)
    xd, wd, sd = to_dev(x, dev), to_dev(w, dev), to_dev(s, dev)
    outs = {}
    for name in ("256x256_w2x4_p", "256x256_w2x4"):
        hx.manifest_clear()
        hx.manifest_enable(True)
        try:
            with pinned(hx, MATMUL_W8, shape, name):
                outs[name] = to_np(hx.matmul(xd, wd, b_layout="nk", col_scale=sd))
            recs = hx.manifest()["records"]
        finally:
            hx.manifest_enable(False)
        assert [r["config"] for r in recs] == [name], recs
    got = outs["256x256_w2x4_p"]
    assert np.array_equal(got.view(np.uint16), outs["256x256_w2x4"].view(np.uint16))
    rows = np.arange(0, M, 97)
    want = oracle.matmul(np.ascontiguousarray(x[rows]), w, b_trans=True, scale_n=s.astype(np.float32))
    g, wv = got[rows].astype(np.float64), want.astype(np.float64)
    assert np.linalg.norm(g - wv) / np.linalg.norm(wv) < 1e-3


def test_swiglu_persistent_equals_one_tile(hx, dev):
    """The FFN's fused gate/up GEMM on the persistent SwiGLU config (T = 2048
    tokens, I = 8192: 512 tiles of 256 x 128, two per workgroup) gives the
    block the same bits as the one-tile config."""
    from test_gpu_ffn import weights
    T, H, I = 2048, 512, 8192
    wg, sg, wu, su, wd, sd = weights(H, I, 930)
    x = rng(931).normal(0, 1, (T, H)).astype(np.float16)
    gamma = rng(932).normal(1, 0.1, H).astype(np.float16)
    Wg = hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev))
    Wu = hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev))
    Wd = hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev))
    outs = {}
    try:
        for name in ("swiglu_256x128_w2x4_p", "swiglu_256x128_w2x4"):
            hx.manifest_clear()
            hx.manifest_enable(True)
            try:
                with pinned(hx, SWIGLU_W8, (T, I, H), name):
                    outs[name] = to_np(hx.swiglu_ffn(to_dev(x, dev), to_dev(gamma, dev), 1e-6, Wg, Wu, Wd))
                recs = hx.manifest()["records"]
            finally:
                hx.manifest_enable(False)
            assert any(r["config"] == name for r in recs), recs
    finally:
        Wg.release(); Wu.release(); Wd.release()
    a, b = outs["swiglu_256x128_w2x4_p"], outs["swiglu_256x128_w2x4"]
    assert np.isfinite(a.astype(np.float32)).all()
    assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    rows = np.array([0, 1, 777, 2047])
    want = oracle.swiglu_ffn(np.ascontiguousarray(x[rows]), gamma, 1e-6, wg, sg, wu, su, wd, sd)
    g, wv = a[rows].astype(np.float64), want.astype(np.float64)
    assert np.linalg.norm(g - wv) / np.linalg.norm(wv) < 2e-3


@pytest.mark.parametrize("op,name", [(MATMUL_F16, "256x256_w2x4_k2"), (MATMUL_F16, "128x128_w2x2_k2"),
                                     (MATMUL_F16, "64x64_w2x2_k4"), (MATMUL_W8, "256x256_w2x4_k2")])
def test_split_merge_in_kernel_is_part_order(hx, dev, op, name):
    """The split output equals RNE((((0 + P0) + P1) + ...) * s) with each
    part's binary32 partial P_q taken from the unsplit config of the same
    tile over that part's K range: the in-kernel merge adds in part order,
    like the merge kernel it replaces."""
    import torch
    cfgs = names_of(hx, op)
    base = name.rsplit("_k", 1)[0]
    assert base in cfgs
    M, N, K = 512, 640, 1984   # edge tiles in N for 256 and 128 wide tiles
    x = rng(940).normal(0, 1, (M, K)).astype(np.float16)
    if op == MATMUL_W8:
        w = i8((N, K), 941)
    else:
        w = rng(941).normal(0, 1, (N, K)).astype(np.float16)
    s = rng(942).uniform(0.5, 2.0, N).astype(np.float32)
    parts = int(name.rsplit("_k", 1)[1])
    # the part length: whole 64-element (128-byte) stages
    per = -(-K // parts)
    ks = -(-per // 64) * 64
    xd, wd = to_dev(x, dev), to_dev(w, dev)
    with pinned(hx, op, (M, N, K), name):
        got = to_np(hx.matmul(xd, wd, b_layout="nk", col_scale=to_dev(s, dev)))
    acc = np.zeros((M, N), np.float32)
    k0 = 0
    while k0 < K:
        k1 = min(K, k0 + ks)
        xp = to_dev(np.ascontiguousarray(x[:, k0:k1]), dev)
        wp = to_dev(np.ascontiguousarray(w[:, k0:k1]), dev)
        with pinned(hx, op, (M, N, k1 - k0), base):
            part = to_np(hx.matmul(xp, wp, b_layout="nk", out_dtype=torch.float32))
        acc = (acc + part).astype(np.float32)
        k0 = k1
    want = (acc * s[None, :]).astype(np.float32).astype(np.float16)
    bad = got.view(np.uint16) != want.view(np.uint16)
    assert not bad.any(), f"{int(bad.sum())} of {bad.size} differ"


def test_clock_probe(hx, dev):
    """One stamp per workgroup of the tiled kernel (256 tiles at 4096^3 with
    the 256 x 256 config), a shader clock between 0.5 and 3 GHz, and nothing
    counted once the probe is off."""
    import torch
    M = N = K = 4096
    a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev)
    b = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev)
    with pinned(hx, GEMM_I8, (M, N, K), "256x256_w2x4"):
        hx.gemm_i8(a, b, b_layout="nk")
        hx.clock_probe(True)
        try:
            for _ in range(3):
                hx.gemm_i8(a, b, b_layout="nk")
            r = hx.clock_read()
        finally:
            hx.clock_probe(False)
        hx.gemm_i8(a, b, b_layout="nk")
    assert r["workgroups"] == 3 * 256, r
    assert 500.0 < r["mhz"] < 3000.0, r
    assert r["workgroup_us"] > 0
    assert hx.clock_read()["workgroups"] == 3 * 256
