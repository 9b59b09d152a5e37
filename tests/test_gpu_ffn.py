"""GPU parity for the SwiGLU FFN composition (scaled down
so the oracle finishes in seconds): RMSNorm -> int8 gate/up GEMMs with
per-channel scales -> SiLU*mul -> int8 down GEMM, every stage rounded to fp16
as separate linalg ops would be.  Both the fused gate/up MFMA path (T > 32)
and the decode path (T <= 32: two GEMVs, with 16-row blocks past 16 tokens;
up to 64 tokens where all three products take the GEMV's four row blocks)
are covered, and the fused gate/up path whose down projection takes the
row blocks (40 tokens at H = 4096, I = 8192: 512 tiles of the gate and up
products take the GEMM)."""
import numpy as np
import pytest

from conftest import assert_close, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu


def weights(H, I, seed):
    r = rng(seed)
    wg = r.integers(-127, 128, (H, I), dtype=np.int8)
    wu = r.integers(-127, 128, (H, I), dtype=np.int8)
    wd = r.integers(-127, 128, (I, H), dtype=np.int8)
    # scales sized so activations stay O(1) through the block
    sg = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    su = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    sd = (r.uniform(0.5, 1.5, H) / (127 * np.sqrt(I / 3))).astype(np.float16)
    return wg, sg, wu, su, wd, sd


@pytest.mark.parametrize("T,H,I", [(256, 512, 1376), (4, 512, 1376), (24, 512, 1376), (40, 512, 1376), (130, 256, 704),
                                   (40, 4096, 11008), (64, 4096, 11008), (40, 4096, 8192)])
def test_swiglu_ffn(hx, dev, T, H, I):
    wg, sg, wu, su, wd, sd = weights(H, I, 300)
    x = rng(301).normal(0, 1, (T, H)).astype(np.float16)
    gamma = rng(302).normal(1, 0.1, H).astype(np.float16)
    Wg = hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev))
    Wu = hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev))
    Wd = hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev))
    try:
        y = hx.swiglu_ffn(to_dev(x, dev), to_dev(gamma, dev), 1e-6, Wg, Wu, Wd)
        got = to_np(y).astype(np.float32)
    finally:
        Wg.release(); Wu.release(); Wd.release()
    want = oracle.swiglu_ffn(x, gamma, 1e-6, wg, sg, wu, su, wd, sd).astype(np.float32)
    # an fp16 rounding flip in an intermediate moves outputs by ~1e-3 relative
    assert_close(got, want, 2e-2, 2e-3, f"swiglu T={T}")
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 2e-3, rel


def test_swiglu_every_config(hx, dev):
    """Every compiled configuration of the fused gate/up (SwiGLU epilogue)
    GEMM family gives the oracle's FFN output (the autotuner may pick any)."""
    T, H, I = 256, 512, 1376
    wg, sg, wu, su, wd, sd = weights(H, I, 310)
    x = rng(311).normal(0, 1, (T, H)).astype(np.float16)
    gamma = rng(312).normal(1, 0.1, H).astype(np.float16)
    want = oracle.swiglu_ffn(x, gamma, 1e-6, wg, sg, wu, su, wd, sd).astype(np.float32)
    Wg = hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev))
    Wu = hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev))
    Wd = hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev))
    n = hx.config_count(5)
    assert n >= 2
    try:
        for cfg in range(n):
            hx.config_select(5, T, I, H, cfg)
            try:
                got = to_np(hx.swiglu_ffn(to_dev(x, dev), to_dev(gamma, dev), 1e-6, Wg, Wu, Wd))
            finally:
                hx.config_select(5, T, I, H, -1)
            assert_close(got.astype(np.float32), want, 2e-2, 2e-3, f"swiglu cfg {cfg}")
    finally:
        Wg.release(); Wu.release(); Wd.release()


def test_swiglu_down_projection_split_k(hx, dev):
    """The down projection through the K-split config (the untuned default at
    the full 2048 x 4096 x 11008 shape): binary32 partials over two halves of
    the intermediate dimension, merged with the down scale, against the
    oracle's composition."""
    T, H, I = 256, 512, 1376
    wg, sg, wu, su, wd, sd = weights(H, I, 320)
    x = rng(321).normal(0, 1, (T, H)).astype(np.float16)
    gamma = rng(322).normal(1, 0.1, H).astype(np.float16)
    want = oracle.swiglu_ffn(x, gamma, 1e-6, wg, sg, wu, su, wd, sd).astype(np.float32)
    Wg = hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev))
    Wu = hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev))
    Wd = hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev))
    names = [hx.config_get(4, i)["name"] for i in range(hx.config_count(4))]
    hx.config_select(4, T, H, I, names.index("256x256_w2x4_k2"))
    hx.manifest_enable(True)
    hx.manifest_clear()
    try:
        got = to_np(hx.swiglu_ffn(to_dev(x, dev), to_dev(gamma, dev), 1e-6, Wg, Wu, Wd)).astype(np.float32)
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
        hx.config_select(4, T, H, I, -1)
        Wg.release(); Wu.release(); Wd.release()
    assert any(rc["config"] == "256x256_w2x4_k2" for rc in recs), \
        [(rc["plan"], rc["config"], rc["reason"]) for rc in recs]
    assert_close(got, want, 2e-2, 2e-3, "swiglu split down projection")
    rel = np.linalg.norm(got - want) / np.linalg.norm(want)
    assert rel < 2e-3, rel


def test_swiglu_ffn_c5_full_size(hx, dev):
    """BASELINE config C5 at its own shape: tokens 2048, hidden 4096,
    intermediate 11008, seeded int8 weights with per-channel fp16 scales,
    gamma N(1, 0.1).  This runs the fused gate/up GEMM over its 688 output
    tiles and the down projection's K = 11008 (split into two binary32 halves
    by the untuned default), checked against the oracle on 512 token rows
    (tokens are independent rows; the first and last are included)."""
    T, H, I = 2048, 4096, 11008
    wg, sg, wu, su, wd, sd = weights(H, I, 330)
    x = rng(331).normal(0, 1, (T, H)).astype(np.float16)
    gamma = rng(332).normal(1, 0.1, H).astype(np.float16)
    Wg = hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev))
    Wu = hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev))
    Wd = hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev))
    hx.manifest_clear()
    hx.manifest_enable(True)
    try:
        y = to_np(hx.swiglu_ffn(to_dev(x, dev), to_dev(gamma, dev), 1e-6, Wg, Wu, Wd)).astype(np.float32)
        recs = hx.manifest()["records"]
    finally:
        hx.manifest_enable(False)
        Wg.release(); Wu.release(); Wd.release()
    plans = {(rc["m"], rc["n"], rc["k"]): rc for rc in recs}
    assert plans[(T, I, H)]["plan"] == "mfma-tiled", plans
    assert plans[(T, H, I)]["plan"] == "mfma-tiled", plans
    # 512 of the 2048 token rows (tokens are independent rows): the first
    # and last of every 256-row tile band plus a seeded sample
    rows = np.unique(np.concatenate([[0, 1, 255, 256, 1023, 1024, 2046, 2047],
                                     rng(333).choice(T, 504, replace=False)]))
    want = oracle.swiglu_ffn(np.ascontiguousarray(x[rows]), gamma, 1e-6, wg, sg, wu, su, wd, sd)
    got = y[rows]
    assert np.isfinite(y).all()
    assert_close(got, want.astype(np.float32), 2e-2, 2e-3, "swiglu C5 sampled rows")
    rel = np.linalg.norm(got - want) / np.linalg.norm(want.astype(np.float32))
    assert rel < 2e-3, rel


@pytest.mark.parametrize("H,I,T", [(512, 2048, 1), (512, 2048, 4), (512, 2048, 16), (512, 2048, 24),
                                   (512, 2048, 32), (4096, 11008, 1), (4096, 11008, 12), (4096, 11008, 24),
                                   (4096, 11008, 40), (4096, 11008, 48)])
def test_swiglu_decode_equals_composition(hx, dev, H, I, T):
    """Decode-sized blocks fuse the gate into the up projection's epilogue
    (RNE(silu(g) * u) on the rounded outputs): the block equals, bit for
    bit, the composition of the public entry points -- RMSNorm, the gate and
    up products, silu_mul, the down product -- also at the north_star
    widths, where the down projection splits K over workgroups from 12
    tokens (two row blocks past 16, four past 32)."""
    import torch
    wg, sg, wu, su, wd, sd = weights(H, I, 700 + T)
    Wg = hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev), layout="kn")
    Wu = hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev), layout="kn")
    Wd = hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev), layout="kn")
    try:
        x = to_dev(rng(710 + T).normal(0, 1, (T, H)).astype(np.float16), dev)
        gamma = to_dev(rng(711).normal(1, 0.1, H).astype(np.float16), dev)
        y = hx.swiglu_ffn(x, gamma, 1e-6, Wg, Wu, Wd)
        h = hx.rms_norm(x, gamma, eps=1e-6)
        a = hx.silu_mul(hx.matmul_resident(h, Wg), hx.matmul_resident(h, Wu))
        want = hx.matmul_resident(a, Wd)
        torch.cuda.synchronize()
        got, ref = to_np(y), to_np(want)
        assert np.isfinite(ref.astype(np.float32)).all()
        assert np.array_equal(got.view(np.uint16), ref.view(np.uint16))
    finally:
        Wg.release(); Wu.release(); Wd.release()
