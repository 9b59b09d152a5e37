"""Tight parity for BASELINE config C3 (W8A16 decode GEMV, M in {1, 4, 16},
N = 11008, K = 4096) and the decode GEMV's K split over workgroups.

* C3 gates, on the resident packed path the bench times and on the in-place
  [K][N] argument path: relative Frobenius error <= 1e-3 against the oracle
  and against a float64 product; every element within one fp16 ulp of the
  oracle's (and of the float64 value's) rounding plus a binary32
  accumulation allowance of 2^-17 * sum_k |x_k w_k| s.  A 0.5% systematic
  error fails both gates (checked on the host).
* The split GEMV's last-arriver merge (partials written by several
  workgroups, the last one to count in adds them in part order): 2000
  back-to-back launches of every split configuration at 16 x 4096 x 11008
  (the FFN's down projection) and 12 x 2048 x 8192, each output compared bit
  for bit with the first, stopping at the first mismatch.
* The split epilogue with the fused SwiGLU gate (decode FFN block whose up
  projection takes a split configuration) equals the composition of the
  public entry points bit for bit.
"""
import numpy as np
import pytest

from conftest import rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu

GEMV = 6  # HX_OP_GEMV: int8 weights, f16 activations


def fp16_ulp(v):
    """The fp16 spacing at |v| (subnormal spacing 2^-24 near zero)."""
    return np.spacing(np.abs(np.asarray(v, np.float64)).astype(np.float16)).astype(np.float64)


def rel_fro(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def c3_gate_failures(got, want, y64, absacc):
    """Names of the C3 gates `got` fails (empty when it passes): relative
    Frobenius <= 1e-3 against the oracle and float64, and per element one
    fp16 ulp (two against float64: its own rounding plus the oracle's) plus
    the binary32 accumulation allowance."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    allow = 2.0 ** -17 * absacc
    bad = []
    if rel_fro(got, want) > 1e-3:
        bad.append(f"rel_fro vs oracle {rel_fro(got, want):.2e}")
    if rel_fro(got, y64) > 1e-3:
        bad.append(f"rel_fro vs float64 {rel_fro(got, y64):.2e}")
    e = np.abs(got - want) > fp16_ulp(want) + allow
    if e.any():
        bad.append(f"{int(e.sum())} elements beyond 1 ulp of the oracle")
    e64 = np.abs(got - y64) > 2 * fp16_ulp(y64) + allow
    if e64.any():
        bad.append(f"{int(e64.sum())} elements beyond 2 ulp of float64")
    return bad


@pytest.fixture(scope="module")
def c3():
    N, K = 11008, 4096
    x = rng(500).normal(0, 1, (16, K)).astype(np.float16)
    w = rng(501).integers(-127, 128, (K, N), dtype=np.int8)      # linalg [K][N]
    s = rng(502).uniform(0.001, 0.02, N).astype(np.float16)
    wt = np.ascontiguousarray(w.T)
    s32 = s.astype(np.float32)
    x64, w64, s64 = x.astype(np.float64), w.astype(np.float64), s32.astype(np.float64)
    ref = {}
    for M in (1, 4, 16):
        want = oracle.matmul(np.ascontiguousarray(x[:M]), wt, b_trans=True, scale_n=s32).astype(np.float64)
        y64 = (x64[:M] @ w64) * s64
        absacc = (np.abs(x64[:M]) @ np.abs(w64)) * s64
        ref[M] = (want, y64, absacc)
    return x, w, wt, s, ref


def test_c3_gates_catch_a_half_percent_error(c3):
    """The gates are not vacuous: the oracle's own output passes them, and
    the same output with a 0.5% systematic error (or one dropped k term's
    worth of error on a tenth of the outputs) fails them."""
    x, w, wt, s, ref = c3
    want, y64, absacc = ref[16]
    assert c3_gate_failures(want, want, y64, absacc) == []
    assert c3_gate_failures(want * 1.005, want, y64, absacc) != []
    dropped = want.copy()
    dropped[:, ::10] -= (x[:, -1:].astype(np.float64) * w[-1, ::10].astype(np.float64)
                         * s[::10].astype(np.float64))
    assert c3_gate_failures(dropped, want, y64, absacc) != []


@pytest.mark.parametrize("M", [1, 4, 16])
def test_c3_resident_tight(hx, dev, c3, M):
    """The bench's path: a registered weight's fragment-packed image with the
    untuned default configuration for this shape."""
    x, w, wt, s, ref = c3
    N, K = wt.shape
    rw = hx.ResidentWeight(to_dev(wt, dev), to_dev(s, dev), layout="nk")
    try:
        got = to_np(hx.matmul_resident(to_dev(np.ascontiguousarray(x[:M]), dev), rw)).astype(np.float64)
    finally:
        rw.release()
    assert c3_gate_failures(got, *ref[M]) == []


@pytest.mark.parametrize("M", [1, 4, 16])
def test_c3_every_config_tight(hx, dev, c3, M):
    """Every compiled decode configuration (the tuner may pin any) under the
    tight gates at M = 1, 4, 16."""
    x, w, wt, s, ref = c3
    N, K = wt.shape
    xt = to_dev(np.ascontiguousarray(x[:M]), dev)
    rw = hx.ResidentWeight(to_dev(wt, dev), to_dev(s, dev), layout="nk")
    try:
        for cfg in range(hx.config_count(GEMV)):
            hx.config_select(GEMV, M, N, K, cfg)
            try:
                got = to_np(hx.matmul_resident(xt, rw)).astype(np.float64)
            finally:
                hx.config_select(GEMV, M, N, K, -1)
            fails = c3_gate_failures(got, *ref[M])
            assert fails == [], (hx.config_get(GEMV, cfg)["name"], fails)
    finally:
        rw.release()


@pytest.mark.parametrize("M", [1, 4, 16])
def test_c3_kn_argument_tight(hx, dev, c3, M):
    """The [K][N] argument weight read in place (no registration)."""
    x, w, wt, s, ref = c3
    y = hx.gemv_w8a16(to_dev(np.ascontiguousarray(x[:M]), dev), to_dev(w, dev), to_dev(s, dev), w_layout="kn")
    assert c3_gate_failures(to_np(y).astype(np.float64), *ref[M]) == []


SPLIT_SHAPES = [(16, 4096, 11008), (12, 2048, 8192), (28, 4096, 11008)]
LAUNCHES = 2000
BATCH = 100


@pytest.mark.parametrize("shape", SPLIT_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_split_gemv_deterministic_at_volume(hx, dev, shape):
    """Each split configuration launched 2000 times back to back (batches of
    100 distinct outputs, no synchronization inside a batch): every output
    equals the first bit for bit.  The parts are added in part order by
    whichever workgroup arrives last, so any lost ordering between a part's
    partial stores and its count shows up as a different sum."""
    import torch
    M, N, K = shape
    g = torch.Generator(device=dev).manual_seed(600 + M)
    w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    s = torch.empty(N, dtype=torch.float16, device=dev).uniform_(0.001, 0.02, generator=g)
    x = torch.randn((M, K), dtype=torch.float16, device=dev, generator=g)
    names = [hx.config_get(GEMV, i)["name"] for i in range(hx.config_count(GEMV))]
    split = [i for i in range(len(names)) if hx.config_get(GEMV, i)["split_k"] > 1]
    assert len(split) >= 5, names
    want = oracle.matmul(x.cpu().numpy(), w.cpu().numpy(), b_trans=True,
                         scale_n=s.float().cpu().numpy()).astype(np.float64)
    rw = hx.ResidentWeight(w, s, layout="nk")
    outs = [torch.empty((M, N), dtype=torch.float16, device=dev) for _ in range(BATCH)]
    try:
        for cfg in split:
            hx.config_select(GEMV, M, N, K, cfg)
            try:
                calls = [hx.bind_matmul_resident(x, rw, y) for y in outs]
                calls[0]()
                first = outs[0].clone()
                assert rel_fro(to_np(first).astype(np.float64), want) < 1e-3, names[cfg]
                ref = first.view(torch.int16).unsqueeze(0)
                for b in range(LAUNCHES // BATCH):
                    for c in calls:
                        c()
                    same = (torch.stack(outs).view(torch.int16) == ref).flatten(1).all(dim=1)
                    if not bool(same.all()):
                        k = int((~same).nonzero()[0])
                        pytest.fail(f"{names[cfg]} {shape}: launch {b * BATCH + k} differs from the first")
            finally:
                hx.config_select(GEMV, M, N, K, -1)
    finally:
        rw.release()


def test_swiglu_decode_split_gate_equals_composition(hx, dev):
    """The decode FFN block with its gated up projection (T = 8, I = 2048,
    H = 8192: M = 8 rows, 128 column tiles, K = 8192) forced onto every
    split configuration and onto the unsplit default: the fused gate in the
    split epilogue gives the composition's bits."""
    import torch
    from test_gpu_ffn import weights
    T, H, I = 8, 8192, 2048
    wg, sg, wu, su, wd, sd = weights(H, I, 800)
    Wg = hx.ResidentWeight(to_dev(wg, dev), to_dev(sg, dev), layout="kn")
    Wu = hx.ResidentWeight(to_dev(wu, dev), to_dev(su, dev), layout="kn")
    Wd = hx.ResidentWeight(to_dev(wd, dev), to_dev(sd, dev), layout="kn")
    names = [hx.config_get(GEMV, i)["name"] for i in range(hx.config_count(GEMV))]
    split = [i for i in range(len(names)) if hx.config_get(GEMV, i)["split_k"] > 1]
    try:
        x = to_dev(rng(801).normal(0, 1, (T, H)).astype(np.float16), dev)
        gamma = to_dev(rng(802).normal(1, 0.1, H).astype(np.float16), dev)
        for cfg in [-1] + split:
            hx.config_select(GEMV, T, I, H, cfg)
            hx.manifest_clear()
            hx.manifest_enable(True)
            try:
                y = hx.swiglu_ffn(x, gamma, 1e-6, Wg, Wu, Wd)
                recs = hx.manifest()["records"]
                h = hx.rms_norm(x, gamma, eps=1e-6)
                a = hx.silu_mul(hx.matmul_resident(h, Wg), hx.matmul_resident(h, Wu))
                want = hx.matmul_resident(a, Wd)
                torch.cuda.synchronize()
            finally:
                hx.manifest_enable(False)
                hx.config_select(GEMV, T, I, H, -1)
            ups = [r for r in recs if (r["m"], r["n"], r["k"]) == (T, I, H)]
            assert ups, recs
            if cfg >= 0:
                # the manifest names the kernel table's entry, the config
                # list prefixes the family ("gemv_")
                assert all(names[cfg] == "gemv_" + r["config"] for r in ups), (names[cfg], ups)
            got, ref = to_np(y), to_np(want)
            assert np.isfinite(ref.astype(np.float32)).all()
            assert np.array_equal(got.view(np.uint16), ref.view(np.uint16)), names[cfg] if cfg >= 0 else "default"
    finally:
        Wg.release(); Wu.release(); Wd.release()
