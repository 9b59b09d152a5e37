"""Rows longer than the four-wave register path holds (more than 16,384
binary32 or 32,768 f16/bf16 elements): the eight-wave single-pass softmax
(16-byte rows up to 16,384 vectors) and the two-pass streaming kernels, the
two-phase form of the reference's online softmax (test/python/triton/
test_online_softmax.py:28-78), for softmax, RMSNorm and LayerNorm, against
float64 arithmetic and the CPU oracle.  Ragged
lengths (element loads), 16-byte rows (vector loads), one row and many,
masked (-inf) logits, strided views."""
import numpy as np
import pytest

from conftest import assert_close, rng, to_dev, to_np
from test_gpu_rows import TOL, make, to_torch, values

import oracle

pytestmark = pytest.mark.gpu

# 16-byte rows up to 16384 vectors, 64 rows or more, take the 8-wave
# single-pass softmax (the norms stream); fewer, ragged or longer rows take
# the two passes
LONG = [(2, 32769, "f16"), (3, 65536, "bf16"), (2, 16385, "f32"), (300, 40000, "f16"),
        (1, 1_000_000, "f32"), (5, 131_088, "f16"), (7, 50_003, "bf16"), (64, 131_072, "f16"),
        (70, 65_536, "f32"), (64, 98_312, "bf16")]


@pytest.mark.parametrize("rows,cols,dtype", LONG, ids=["-".join(map(str, c)) for c in LONG])
def test_long_rows_three_ops(hx, dev, rows, cols, dtype):
    bf = dtype == "bf16"
    rtol, atol = TOL[dtype]
    xh, xf = make(dtype, (rows, cols), seed=cols + rows)
    y = values(to_np(hx.softmax(to_torch(xh, dtype, dev))), dtype)
    assert_close(y, values(oracle.softmax(xh, bf16=bf), dtype), rtol, atol, "softmax")
    # long rows put most outputs far below atol: bound the relative Frobenius
    # error against the exact softmax of the same inputs, at about three
    # times what correctly rounded outputs give (f16 3.7e-4, bf16 2.0e-3,
    # f32 1e-6 at these shapes; the oracle's own sequential binary32 sum is
    # only good to 9e-4 at 10^6 columns)
    x64 = xf.astype(np.float64)
    e = np.exp(x64 - x64.max(axis=1, keepdims=True))
    p = e / e.sum(axis=1, keepdims=True)
    rel = np.linalg.norm(y.astype(np.float64) - p) / np.linalg.norm(p)
    assert rel <= {"f16": 1.5e-3, "bf16": 6e-3, "f32": 1e-5}[dtype], rel
    # every row is a distribution: its sum is one to the outputs' rounding
    # (about sqrt(cols) half-ulps of the largest outputs)
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=2e-2 if dtype != "f32" else 1e-4)
    # the norms against float64 math on the same inputs, and against the
    # oracle, whose sequential binary32 sums drift with the row length (2e-4
    # relative, 1.3e-4 absolute in LayerNorm outputs at 10^6 binary32
    # columns: any summation order is the reference's semantics, so the
    # oracle bound there covers the order)
    ortol, oatol = (1e-3, 1e-3) if (dtype == "f32" and cols > (1 << 17)) else (rtol, atol)
    gh, gf = make(dtype, (cols,), sigma=0.1, mean=1.0, seed=cols)
    y = values(to_np(hx.rms_norm(to_torch(xh, dtype, dev), to_torch(gh, dtype, dev), eps=1e-6)), dtype)
    x64 = xf.astype(np.float64)
    exact = x64 / np.sqrt((x64 * x64).mean(axis=1, keepdims=True) + 1e-6) * gf
    assert_close(y, exact, rtol, atol, "rmsnorm vs float64")
    assert_close(y, values(oracle.rmsnorm(xh, gh, 1e-6, bf16=bf), dtype), ortol, oatol, "rmsnorm vs oracle")
    xl, xlf = make(dtype, (rows, cols), seed=cols + 1, mean=0.5)
    wh, wf = make(dtype, (cols,), sigma=0.2, mean=1.0, seed=cols + 2)
    bh, bfv = make(dtype, (cols,), sigma=0.2, seed=cols + 3)
    y, mean, rstd = hx.layer_norm(to_torch(xl, dtype, dev), to_torch(wh, dtype, dev), to_torch(bh, dtype, dev),
                                  eps=1e-5, return_stats=True)
    y = values(to_np(y), dtype)
    l64 = xlf.astype(np.float64)
    mu = l64.mean(axis=1)
    rs = 1.0 / np.sqrt(((l64 - mu[:, None]) ** 2).mean(axis=1) + 1e-5)
    assert_close(y, (l64 - mu[:, None]) * rs[:, None] * wf + bfv, rtol, atol, "layernorm vs float64")
    assert_close(to_np(mean), mu, 1e-5, 1e-5, "mean vs float64")
    assert_close(to_np(rstd), rs, 1e-4, 1e-5, "rstd vs float64")
    want, wm, wr = oracle.layernorm(xl, wh, bh, 1e-5, bf16=bf)
    assert_close(y, values(want, dtype), ortol, oatol, "layernorm vs oracle")


def test_long_softmax_masked_logits(hx, dev):
    """-inf logits (masked vocabulary entries) contribute zero; a row masked
    everywhere but one entry puts all its mass there."""
    rows, cols = 4, 100_000
    r = rng(91)
    x = r.normal(0, 3, (rows, cols)).astype(np.float16)
    x[r.random((rows, cols)) < 0.3] = -np.inf
    x[3, :] = -np.inf
    x[3, 77_777] = 1.5
    got = to_np(hx.softmax(to_dev(x, dev))).astype(np.float32)
    want = oracle.softmax(x).astype(np.float32)
    assert_close(got, want, 1e-2, 1e-3, "masked softmax")
    assert (got[x == -np.inf] == 0).all()
    assert got[3, 77_777] == 1.0 and np.count_nonzero(got[3]) == 1


def test_long_rows_strided_views(hx, dev):
    """Row views into wider buffers (outer stride > cols): only the view is
    read and written."""
    import torch
    rows, cols, pad = 6, 40_000, 24
    xh, _ = make("f16", (rows, cols + pad), seed=17)
    xt = to_dev(xh, dev)[:, :cols]
    out = torch.full((rows, cols + pad), 5.0, dtype=torch.float16, device=dev)
    hx.softmax(xt, out=out[:, :cols])
    got = to_np(out)
    want = oracle.softmax(np.ascontiguousarray(xh[:, :cols]))
    assert_close(got[:, :cols].astype(np.float32), want.astype(np.float32), 1e-2, 1e-3, "strided long softmax")
    assert (got[:, cols:] == np.float16(5.0)).all(), "wrote outside the view"


def test_online_softmax_reference_case(hx, dev):
    """The reference's online-softmax test configuration: 128 x 128 f32 from
    torch.rand, atol 1e-5 (test_online_softmax.py:18-20, 83-98)."""
    x = rng(92).random((128, 128)).astype(np.float32)
    got = to_np(hx.softmax(to_dev(x, dev)))
    want = oracle.softmax(x)
    assert np.abs(got - want).max() <= 1e-5
