"""GPU parity: softmax / RMSNorm / LayerNorm / SiLU*mul against the oracle.

Tolerances: fp16 / bf16 outputs within rtol 1e-2, atol 1e-3 (BASELINE.json
north star; the reference's own softmax gate is atol 1e-3 for fp16,
test/python/triton/test_softmax.py:27-28); f32 within rtol 1e-4, atol 1e-5
(test_layer_norm.py:22, test_softmax.py:27).  The fp32 results differ from the
oracle only by reduction order and the hardware exp2 / rsqrt-free chain.
"""
import numpy as np
import pytest

from conftest import assert_close, bf16_from_f32, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu

TOL = {"f16": (1e-2, 1e-3), "bf16": (1e-2, 1e-3), "f32": (1e-4, 1e-5)}


def make(dtype, shape, sigma=2.0, seed=0, mean=0.0):
    """Host array in the test dtype (bf16 as uint16 bits) + its f32 values."""
    x = rng(seed).normal(mean, sigma, shape).astype(np.float32)
    if dtype == "f16":
        h = x.astype(np.float16)
        return h, h.astype(np.float32)
    if dtype == "bf16":
        b = bf16_from_f32(x)
        return b, oracle.bf16_bits_to_f32(b)
    return x, x


def to_torch(h, dtype, dev):
    import torch
    t = to_dev(h.view(np.int16) if dtype == "bf16" else h, dev)
    return t.view(torch.bfloat16) if dtype == "bf16" else t


def values(arr, dtype):
    if dtype == "bf16":
        return oracle.bf16_bits_to_f32(arr)
    return np.asarray(arr, np.float32)


SHAPES = [(8192, 4096), (128, 128), (127, 513), (27, 8192), (3, 1), (5, 16384), (64, 100)]


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_softmax(hx, dev, dtype, shape):
    xh, _ = make(dtype, shape, seed=1)
    y = hx.softmax(to_torch(xh, dtype, dev))
    want = oracle.softmax(xh, bf16=(dtype == "bf16"))
    rtol, atol = TOL[dtype]
    got = values(to_np(y), dtype)
    assert_close(got, values(want, dtype), rtol, atol, f"softmax {dtype} {shape}")
    # rows of a softmax sum to one (to the output's rounding)
    assert np.allclose(got.astype(np.float64).sum(axis=1), 1.0, atol=2e-2 if dtype != "f32" else 1e-4)


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_rmsnorm(hx, dev, dtype, shape):
    xh, _ = make(dtype, shape, seed=2)
    gh, _ = make(dtype, (shape[1],), sigma=0.1, mean=1.0, seed=3)
    y = hx.rms_norm(to_torch(xh, dtype, dev), to_torch(gh, dtype, dev), eps=1e-6)
    want = oracle.rmsnorm(xh, gh, 1e-6, bf16=(dtype == "bf16"))
    rtol, atol = TOL[dtype]
    assert_close(values(to_np(y), dtype), values(want, dtype), rtol, atol, f"rmsnorm {dtype} {shape}")


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: f"{s[0]}x{s[1]}")
def test_layernorm(hx, dev, dtype, shape):
    xh, _ = make(dtype, shape, seed=4, mean=0.5)
    wh, _ = make(dtype, (shape[1],), sigma=0.2, mean=1.0, seed=5)
    bh, _ = make(dtype, (shape[1],), sigma=0.2, seed=6)
    y, mean, rstd = hx.layer_norm(to_torch(xh, dtype, dev), to_torch(wh, dtype, dev),
                                  to_torch(bh, dtype, dev), eps=1e-5, return_stats=True)
    want, wm, wr = oracle.layernorm(xh, wh, bh, 1e-5, bf16=(dtype == "bf16"))
    rtol, atol = TOL[dtype]
    assert_close(values(to_np(y), dtype), values(want, dtype), rtol, atol, f"layernorm {dtype} {shape}")
    assert_close(to_np(mean), wm, 1e-5, 1e-5, "mean")
    assert_close(to_np(rstd), wr, 1e-4, 1e-5, "rstd")


def test_rmsnorm_no_gamma_and_strided_rows(hx, dev):
    """gamma=None is the identity; an outer stride > cols (a view into a
    wider buffer) reads and writes only the view."""
    import torch
    x, _ = make("f16", (64, 4096 + 64), seed=7)
    xt = to_dev(x, dev)[:, :4096]
    out_full = torch.full((64, 4096 + 64), 7.0, dtype=torch.float16, device=dev)
    hx.rms_norm(xt, None, eps=1e-6, out=out_full[:, :4096])
    want = oracle.rmsnorm(np.ascontiguousarray(x[:, :4096]), None, 1e-6)
    got = to_np(out_full)
    assert_close(got[:, :4096].astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, "strided rmsnorm")
    assert (got[:, 4096:] == np.float16(7.0)).all(), "wrote outside the view"


def test_softmax_reference_shape_against_torch(hx, dev):
    """The reference test's own oracle and gate: torch softmax, atol 1e-3
    (test/python/triton/test_softmax.py:88-93), at its 128x128 shape."""
    import torch
    x = torch.rand(128, 128, dtype=torch.float16, generator=torch.Generator().manual_seed(0))
    y = hx.softmax(x.to(dev)).cpu()
    ref = torch.nn.functional.softmax(x.float(), dim=1).half()
    assert torch.allclose(y, ref, atol=1e-3)


def test_silu_mul(hx, dev):
    g, _ = make("f16", (64, 11008), sigma=2.0, seed=8)
    u, _ = make("f16", (64, 11008), sigma=1.0, seed=9)
    y = hx.silu_mul(to_dev(g, dev), to_dev(u, dev))
    want = oracle.silu_mul(g, u)
    assert_close(to_np(y).astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, "silu_mul")
    # odd width takes the element path
    y2 = hx.silu_mul(to_dev(g[:, :1001].copy(), dev), to_dev(u[:, :1001].copy(), dev))
    assert_close(to_np(y2).astype(np.float32), want[:, :1001].astype(np.float32), 1e-2, 1e-3, "silu_mul odd")


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_softmax_c4_relative(hx, dev, dtype):
    """C4 softmax (8192 x 4096, N(0, 2)) checked in relative terms: most
    outputs are ~1e-4 or smaller, where the absolute gate above says little.
    Every output in the normal range of the type must agree with the oracle
    to a few ulps of relative error, subnormal fp16 outputs to two subnormal
    ulps, and the whole matrix to a relative Frobenius error of 1e-3 (a 1%
    error in exp, or a row sum off by 1%, fails all three)."""
    xh, _ = make(dtype, (8192, 4096), seed=11)
    got = values(to_np(hx.softmax(to_torch(xh, dtype, dev))), dtype).astype(np.float64)
    want = values(oracle.softmax(xh, bf16=(dtype == "bf16")), dtype).astype(np.float64)
    tiny = 2.0 ** -14 if dtype == "f16" else 2.0 ** -126   # smallest normal of the type
    ulp_rel = 2.0 ** -10 if dtype == "f16" else 2.0 ** -7  # one ulp, relative, at worst
    normal = want >= tiny
    assert normal.mean() > 0.3, normal.mean()  # ~38% of fp16 outputs are normal numbers
    err = np.abs(got - want)
    assert (err[normal] <= 2 * ulp_rel * want[normal]).all(), float((err[normal] / want[normal]).max())
    if dtype == "f16":
        assert (err[~normal] <= 2.0 ** -23).all(), float(err[~normal].max())
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 1e-3, rel
    # each row's mass is 1 to within the outputs' own rounding
    assert np.abs(got.sum(axis=1) - 1.0).max() < (2e-3 if dtype == "f16" else 2e-2)



def ulp_of(v, dtype):
    """Spacing of the output type at |v| (fp16 via numpy, subnormals
    included; bf16 as 2^(e - 7), with its smallest normal's spacing below)."""
    a = np.abs(np.asarray(v, np.float64))
    if dtype == "f16":
        return np.spacing(a.astype(np.float16)).astype(np.float64)
    e = np.floor(np.log2(np.maximum(a, 2.0 ** -126)))
    return 2.0 ** (e - 7)


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_rmsnorm_c4_ulps(hx, dev, dtype):
    """C4 RMSNorm (8192 x 4096, x N(0, 2), gamma N(1, 0.1), eps 1e-6): every
    output within 2 ulps of the type of the oracle's, and a relative
    Frobenius error against float64 below 1e-3 (fp16; bf16's own rounding
    alone gives about 1.6e-3, so 4e-3 there).  The two differ only in the
    order of the binary32 sum of squares, so a dropped term, a wrong eps or
    a 0.2% scale error (rstd off by one part in 500; 2% for bf16) fails."""
    xh, xf = make(dtype, (8192, 4096), seed=12)
    gh, gf = make(dtype, (4096,), sigma=0.1, mean=1.0, seed=13)
    got = values(to_np(hx.rms_norm(to_torch(xh, dtype, dev), to_torch(gh, dtype, dev), eps=1e-6)),
                 dtype).astype(np.float64)
    want = values(oracle.rmsnorm(xh, gh, 1e-6, bf16=(dtype == "bf16")), dtype).astype(np.float64)
    x64 = xf.astype(np.float64)
    y64 = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6) * gf.astype(np.float64)
    err = np.abs(got - want)
    lim = 2 * ulp_of(want, dtype)
    assert (err <= lim).all(), (int((err > lim).sum()), float((err / np.maximum(lim, 1e-30)).max()))
    rel = np.linalg.norm(got - y64) / np.linalg.norm(y64)
    assert rel < (1e-3 if dtype == "f16" else 4e-3), rel
    # the gate is not vacuous: the oracle scaled by 1.002 (fp16) or 1.02
    # (bf16, whose two ulps span up to 1.6%) fails it
    bump = 1.002 if dtype == "f16" else 1.02
    assert not (np.abs(want * bump - want) <= lim).all()


@pytest.mark.parametrize("dtype", ["f16", "bf16"])
def test_layernorm_c4_ulps(hx, dev, dtype):
    """LayerNorm at the C4 shape: every output within 2 ulps of the oracle's
    plus a binary32 allowance relative to the terms it adds (y = t + b with
    t = (x - mean) * rstd * w can cancel) and to the mean's own rounding, relative Frobenius against float64
    below 1e-3 (bf16: 4e-3), and the mean / rstd outputs as in
    test_layernorm."""
    xh, xf = make(dtype, (8192, 4096), seed=14, mean=0.5)
    wh, wf = make(dtype, (4096,), sigma=0.2, mean=1.0, seed=15)
    bh, bf = make(dtype, (4096,), sigma=0.2, seed=16)
    y, mean, rstd = hx.layer_norm(to_torch(xh, dtype, dev), to_torch(wh, dtype, dev), to_torch(bh, dtype, dev),
                                  eps=1e-5, return_stats=True)
    got = values(to_np(y), dtype).astype(np.float64)
    want, wm, wr = oracle.layernorm(xh, wh, bh, 1e-5, bf16=(dtype == "bf16"))
    want = values(want, dtype).astype(np.float64)
    x64 = xf.astype(np.float64)
    mu = x64.mean(axis=1, keepdims=True)
    rs = 1.0 / np.sqrt(((x64 - mu) ** 2).mean(axis=1, keepdims=True) + 1e-5)
    t64 = (x64 - mu) * rs * wf.astype(np.float64)
    y64 = t64 + bf.astype(np.float64)
    err = np.abs(got - want)
    # allowance: binary32 rounding of the terms, and the mean's own binary32
    # error (a sequential sum of 4096 terms, ~1e-6 here) carried through
    # rstd * w
    lim = (2 * ulp_of(want, dtype) + 2.0 ** -20 * (np.abs(t64) + np.abs(bf.astype(np.float64)))
           + 2.0 ** -17 * rs * np.abs(wf.astype(np.float64)))
    assert (err <= lim).all(), (int((err > lim).sum()), float((err / lim).max()))
    rel = np.linalg.norm(got - y64) / np.linalg.norm(y64)
    assert rel < (1e-3 if dtype == "f16" else 4e-3), rel
    assert_close(to_np(mean), wm, 1e-5, 1e-5, "mean")
    assert_close(to_np(rstd), wr, 1e-4, 1e-5, "rstd")


# (rows, cols): odd row counts around the streaming grid, fewer rows than the
# grid, 2 / 4 / 8 / 16 vectors per lane in f16, a row the streaming form does
# not take (1000 columns), and a strided view
ROW_CFG_SHAPES = [(2085, 4096), (3, 4096), (1030, 8192), (517, 16384), (300, 32768), (700, 1000)]
DT_CODE = {"f16": 1, "bf16": 2, "f32": 3}


@pytest.mark.parametrize("dtype", ["f16", "bf16", "f32"])
@pytest.mark.parametrize("op", ["softmax", "rmsnorm", "layernorm"])
def test_row_configs_bit_equal(hx, dev, op, dtype):
    """Every row configuration (one row per workgroup, the streaming form at
    2, 4 and 8 workgroups per CU), pinned through hx_config_select, writes
    the same bits as the one-row form -- outputs, and LayerNorm's mean and
    rstd -- and the one-row form agrees with the oracle; views whose outer
    stride exceeds the row are read and written only inside the view."""
    import torch
    fam = {"softmax": 9, "rmsnorm": 10, "layernorm": 11}[op]
    n_cfg = hx.config_count(fam)
    for rows, cols in ROW_CFG_SHAPES + [(2100, 4096 + 64)]:
        strided = cols == 4096 + 64
        xh, _ = make(dtype, (rows, cols), seed=rows + cols, mean=0.25)
        gh, _ = make(dtype, (cols,), sigma=0.2, mean=1.0, seed=11)
        bh, _ = make(dtype, (cols,), sigma=0.2, seed=12)
        xt = to_torch(xh, dtype, dev)
        width = cols - 64 if strided else cols
        if strided:
            xt = xt[:, :width]
            gh, bh = gh[:width], bh[:width]
        gt, bt = to_torch(np.ascontiguousarray(gh), dtype, dev), to_torch(np.ascontiguousarray(bh), dtype, dev)

        def run(idx):
            hx.config_select(fam, rows, width, DT_CODE[dtype], idx)
            try:
                full = torch.full((rows, cols), 3.0, dtype=xt.dtype, device=dev)
                y = full[:, :width]
                stats = ()
                if op == "softmax":
                    hx.softmax(xt, out=y)
                elif op == "rmsnorm":
                    hx.rms_norm(xt, gt, eps=1e-6, out=y)
                else:
                    _, m, r = hx.layer_norm(xt, gt, bt, eps=1e-5, out=y, return_stats=True)
                    stats = (to_np(m), to_np(r))
                return to_np(full), stats
            finally:
                hx.config_select(fam, rows, width, DT_CODE[dtype], -1)

        base, base_stats = run(0)
        if strided:
            assert (values(base[:, width:], dtype) == 3.0).all(), "wrote outside the view"
        for idx in range(1, n_cfg):
            got, stats = run(idx)
            name = hx.config_get(fam, idx)["name"]
            assert np.array_equal(got.view(np.uint8), base.view(np.uint8)), (op, dtype, rows, cols, name)
            for a, b in zip(stats, base_stats):
                assert np.array_equal(a.view(np.uint8), b.view(np.uint8)), (op, dtype, rows, cols, name, "stats")
        if rows * width <= 2100 * 4096 and not strided:
            xs = np.ascontiguousarray(xh)
            if op == "softmax":
                want = oracle.softmax(xs, bf16=(dtype == "bf16"))
            elif op == "rmsnorm":
                want = oracle.rmsnorm(xs, gh, 1e-6, bf16=(dtype == "bf16"))
            else:
                want = oracle.layernorm(xs, gh, bh, 1e-5, bf16=(dtype == "bf16"))[0]
            rtol, atol = TOL[dtype]
            assert_close(values(base, dtype), values(want, dtype), rtol, atol, f"{op} {dtype} {rows}x{cols}")


def test_row_default_configs(hx, dev):
    """The untuned choice: the norms stream at 4 KiB-or-longer rows once there
    are two rows per workgroup of the grid; softmax runs one row per
    workgroup."""
    cus = __import__("torch").cuda.get_device_properties(0).multi_processor_count
    look = lambda fam, r, c, dt=1: hx.config_get(fam, hx.config_lookup(fam, r, c, dt))["name"]  # noqa: E731
    assert look(9, 8192, 4096) == "row"
    assert look(10, 8192, 4096) == "stream_4" and look(11, 8192, 4096) == "stream_4"
    assert look(10, 2 * 4 * cus - 1, 4096) == "row"
    assert look(10, 4096, 8192) == "stream_2" and look(11, 4096, 32768) == "stream_2"
    assert look(10, 8192, 1024) == "row"      # 2 KiB rows: one wave per row
    assert look(10, 8192, 4096, 3) == "stream_2"  # f32: 16 KiB rows
