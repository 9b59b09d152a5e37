"""Pins for the CPU oracle (oracle/hx_oracle.c).  Every oracle function is
checked against something that does not share its code: numpy / torch-CPU
library routines, closed forms, invariants or brute force -- chosen so that
a plausible mistake (a dropped term, a wrong order, a transposed operand)
fails one of them.  The reference ships no numeric fixtures for this path
(its device tests draw torch.rand at run time), so the reference tests'
own oracles and tolerances are reproduced at their shapes
(test/python/triton/test_softmax.py, test_rms_norm.py, test_layer_norm.py),
plus small committed fixtures under tests/golden/."""
import json
from pathlib import Path

import numpy as np
import pytest

import oracle
from conftest import assert_close, rng

GOLDEN = Path(__file__).resolve().parent / "golden"


# --------------------------------------------------------------------------- #
# Conversions
# --------------------------------------------------------------------------- #

def test_f32_to_f16_matches_numpy_rne():
    specials = np.array([0.0, -0.0, 1.0, -1.0, 65504.0, 65519.996, 65520.0, 65536.0, 1e9, -1e9,
                         np.inf, -np.inf, 2.0 ** -14, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                         2.0 ** -25 * 1.0000001, 2.0 ** -14 - 2.0 ** -25, 1e-8, 5.96e-8, 0.1, 1 / 3],
                        dtype=np.float32)
    # ties: exactly halfway between two f16 values, at several binades
    base = np.arange(1024, 2048, dtype=np.float32)
    ties = np.concatenate([(base + 0.5) * 2.0 ** e for e in (-24, -20, -10, 0, 5)]).astype(np.float32)
    bits = rng(0).integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    rand = bits.view(np.float32)
    rand = rand[np.isfinite(rand)]
    for x in (specials, ties, rand):
        got = oracle.f32_to_f16_bits(x)
        want = x.astype(np.float16).view(np.uint16)
        assert np.array_equal(got, want)
    nan = oracle.f32_to_f16_bits(np.array([np.nan], np.float32))
    assert np.isnan(nan.view(np.float16)).all()


def test_f16_to_f32_all_65536_patterns():
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = oracle.f16_bits_to_f32(h)
    want = h.view(np.float16).astype(np.float32)
    finite = np.isfinite(want)
    assert np.array_equal(got[finite].view(np.uint32), want[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(want))
    assert np.array_equal(np.isinf(got), np.isinf(want))


def test_f32_to_bf16_matches_torch_rne():
    torch = pytest.importorskip("torch")
    bits = rng(1).integers(0, 2 ** 32, 1 << 20, dtype=np.uint64).astype(np.uint32)
    x = bits.view(np.float32)
    x = x[~np.isnan(x)]
    got = oracle.f32_to_bf16_bits(x)
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(got, want)
    assert np.array_equal(oracle.bf16_bits_to_f32(got).view(np.uint32),
                          torch.from_numpy(want.view(np.int16)).view(torch.bfloat16).float().numpy().view(np.uint32))


# --------------------------------------------------------------------------- #
# int8 GEMM
# --------------------------------------------------------------------------- #

def test_gemm_i8_brute_force_small():
    a = rng(2).integers(-127, 128, (5, 3), dtype=np.int8)
    b = rng(3).integers(-127, 128, (3, 7), dtype=np.int8)
    want = [[sum(int(a[i, k]) * int(b[k, j]) for k in range(3)) for j in range(7)] for i in range(5)]
    assert oracle.gemm_i8_i32(a, b).tolist() == want


@pytest.mark.parametrize("shape", [(64, 64, 64), (37, 129, 260), (1, 4096, 512), (200, 3, 1000)])
def test_gemm_i8_matches_numpy_int64(shape):
    M, N, K = shape
    a = rng(4).integers(-127, 128, (M, K), dtype=np.int8)
    b = rng(5).integers(-127, 128, (K, N), dtype=np.int8)
    want = a.astype(np.int64) @ b.astype(np.int64)
    got = oracle.gemm_i8_i32(a, b)
    assert np.array_equal(got, want)
    assert np.array_equal(oracle.gemm_i8_i32(a, np.ascontiguousarray(b.T), b_trans=True), want)
    # negative control: the transposed-operand mistake is visible to this check
    if M == N == K:
        assert not np.array_equal(got, a.astype(np.int64) @ b.T.astype(np.int64))


def test_gemm_i8_closed_forms():
    K = 4096
    a = np.full((3, K), 127, np.int8)
    b = np.full((K, 2), -127, np.int8)
    assert (oracle.gemm_i8_i32(a, b) == -K * 127 * 127).all()        # no int32 overflow at K=4096
    a = np.full((2, K), -127, np.int8)
    assert (oracle.gemm_i8_i32(a, np.full((K, 2), -127, np.int8)) == K * 127 * 127).all()
    x = rng(6).integers(-127, 128, (9, 9), dtype=np.int8)
    assert np.array_equal(oracle.gemm_i8_i32(x, np.eye(9, dtype=np.int8)), x.astype(np.int32))
    u = rng(7).integers(-127, 128, (8, 1), dtype=np.int8)
    v = rng(8).integers(-127, 128, (1, 6), dtype=np.int8)
    assert np.array_equal(oracle.gemm_i8_i32(u, v), np.outer(u.astype(np.int32), v.astype(np.int32)))


def test_dequant_matches_numpy_binary32_bitwise():
    c = rng(9).integers(-66_064_384, 66_064_385, (64, 96), dtype=np.int64).astype(np.int32)
    sa = rng(10).uniform(0.001, 0.02, 64).astype(np.float32)
    sb = rng(11).uniform(0.001, 0.02, 96).astype(np.float32)
    want = ((c.astype(np.float32) * sa[:, None]).astype(np.float32) * sb[None, :]).astype(np.float16)
    got = oracle.dequant_i32_f16(c, sa, sb)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))
    # dropping the column scale is caught
    assert not np.array_equal(oracle.dequant_i32_f16(c, sa, None).view(np.uint16), want.view(np.uint16))
    # small accumulators land in the fp16 subnormal range and still agree
    tiny = rng(12).integers(-3, 4, (8, 8)).astype(np.int32)
    want_t = ((tiny.astype(np.float32) * sa[:8, None]) * sb[None, :8]).astype(np.float16)
    assert np.array_equal(oracle.dequant_i32_f16(tiny, sa[:8], sb[:8]).view(np.uint16), want_t.view(np.uint16))


# --------------------------------------------------------------------------- #
# Floating matmul
# --------------------------------------------------------------------------- #

def _bound(a, b):
    """binary32 accumulation bound K*eps*sum|a||b| plus the output rounding."""
    K = a.shape[1]
    return K * 2.0 ** -24 * (np.abs(a).astype(np.float64) @ np.abs(b).astype(np.float64))


def test_matmul_f16_within_accumulation_bound():
    a = rng(13).uniform(-1, 1, (48, 300)).astype(np.float16)
    b = rng(14).uniform(-1, 1, (300, 80)).astype(np.float16)
    exact = a.astype(np.float64) @ b.astype(np.float64)
    got32 = oracle.matmul(a, b, out_dtype=np.float32).astype(np.float64)
    assert (np.abs(got32 - exact) <= _bound(a, b) + 1e-12).all()
    got16 = oracle.matmul(a, b).astype(np.float64)
    assert np.array_equal(got16, got32.astype(np.float32).astype(np.float16).astype(np.float64))
    assert np.array_equal(oracle.matmul(a, np.ascontiguousarray(b.T), b_trans=True), oracle.matmul(a, b))


def test_matmul_identity_is_exact():
    a = rng(15).normal(0, 3, (17, 64)).astype(np.float16)
    eye = np.eye(64, dtype=np.float16)
    assert np.array_equal(oracle.matmul(a, eye).view(np.uint16), a.view(np.uint16))


def test_matmul_bf16_and_w8a16():
    a32 = rng(16).uniform(-1, 1, (20, 96)).astype(np.float32)
    b32 = rng(17).uniform(-1, 1, (96, 24)).astype(np.float32)
    ab, bb = oracle.f32_to_bf16_bits(a32), oracle.f32_to_bf16_bits(b32)
    got = oracle.bf16_bits_to_f32(oracle.matmul(ab, bb, a_bf16=True, b_bf16=True, out_bf16=True))
    exact = oracle.bf16_bits_to_f32(ab).astype(np.float64) @ oracle.bf16_bits_to_f32(bb).astype(np.float64)
    assert_close(got, exact, 2 ** -8, 1e-6, "bf16 matmul")
    x = rng(18).normal(0, 1, (4, 256)).astype(np.float16)
    w = rng(19).integers(-127, 128, (256, 40), dtype=np.int8)
    s = rng(20).uniform(0.001, 0.02, 40).astype(np.float32)
    exact = (x.astype(np.float64) @ w.astype(np.float64)) * s.astype(np.float64)
    got = oracle.matmul(x, w, scale_n=s).astype(np.float64)
    assert_close(got, exact, 1e-3, 1e-4, "w8a16")
    assert not np.allclose(oracle.matmul(x, w).astype(np.float64), exact, rtol=1e-2)  # scale not dropped


def test_matmul_residual_term():
    a = rng(21).uniform(-1, 1, (16, 32)).astype(np.float16)
    b = rng(22).uniform(-1, 1, (32, 16)).astype(np.float16)
    r = rng(23).normal(0, 1, (16, 16)).astype(np.float32)
    got = oracle.matmul(a, b, residual=r, out_dtype=np.float32)
    want = oracle.matmul(a, b, out_dtype=np.float32) + r
    assert np.array_equal(got, want)


def test_matmul_scale_and_residual_together():
    """Both optional terms at once: out = (A.B) * s[j] + R[i, j], the scale
    applied to the product only (the reference's per-channel read-out scale
    followed by the residual add, MatmulToHmxPass.cpp:100-121,
    HMXLayout.c:868-999).  Checked against an independent float64
    composition within the binary32 accumulation bound plus the final
    roundings; the swapped order (A.B + R) * s must fail the same gate."""
    a = rng(24).uniform(-1, 1, (24, 200)).astype(np.float16)
    b = rng(25).uniform(-1, 1, (200, 40)).astype(np.float16)
    s = rng(26).uniform(0.5, 4.0, 40).astype(np.float32)
    r = rng(27).normal(0, 3, (24, 40)).astype(np.float16)
    ab = a.astype(np.float64) @ b.astype(np.float64)
    want = ab * s.astype(np.float64) + r.astype(np.float64)
    bound = _bound(a, b) * s.astype(np.float64) + 2.0 ** -23 * (np.abs(ab * s) + np.abs(want))
    got32 = oracle.matmul(a, b, scale_n=s, residual=r, out_dtype=np.float32).astype(np.float64)
    assert (np.abs(got32 - want) <= bound + 1e-12).all()
    got16 = oracle.matmul(a, b, scale_n=s, residual=r).astype(np.float64)
    assert np.array_equal(got16, got32.astype(np.float32).astype(np.float16).astype(np.float64))
    swapped = (ab + r.astype(np.float64)) * s.astype(np.float64)
    assert not (np.abs(got32 - swapped) <= bound + 1e-12).all(), "gate cannot tell the order apart"
    # the int8-weight form (W8A16 with a residual) through the same path
    w = rng(28).integers(-127, 128, (200, 40), dtype=np.int8)
    got = oracle.matmul(a, w, scale_n=s, residual=r, out_dtype=np.float32).astype(np.float64)
    aw = a.astype(np.float64) @ w.astype(np.float64)
    want_w = aw * s + r.astype(np.float64)
    bound_w = _bound(a, w) * s + 2.0 ** -23 * (np.abs(aw * s) + np.abs(want_w))
    assert (np.abs(got - want_w) <= bound_w + 1e-12).all()


@pytest.mark.parametrize("trans", [False, True])
def test_matmul_column_split_is_bit_identical(trans):
    """The column-split form (host threads over output columns, for the
    few-row CPU baselines) sums each element in the same k order, so it is
    bit-identical to the row form, with scale and residual."""
    x = rng(29).normal(0, 1, (5, 300)).astype(np.float16)
    w = rng(30).integers(-127, 128, (300, 1000), dtype=np.int8)
    s = rng(31).uniform(0.001, 0.02, 1000).astype(np.float32)
    r = rng(32).normal(0, 1, (5, 1000)).astype(np.float16)
    wb = np.ascontiguousarray(w.T) if trans else w
    want = oracle.matmul(x, wb, b_trans=trans, scale_n=s, residual=r)
    got = oracle.matmul(x, wb, b_trans=trans, scale_n=s, residual=r, split_cols=True)
    assert np.array_equal(got.view(np.uint16), want.view(np.uint16))


# --------------------------------------------------------------------------- #
# Row reductions
# --------------------------------------------------------------------------- #

def _softmax64(x):
    x = x.astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    return e / e.sum(axis=1, keepdims=True)


def test_softmax_vs_float64_and_invariants():
    x = rng(24).normal(0, 2, (64, 4096)).astype(np.float32)
    y = oracle.softmax(x)
    assert_close(y, _softmax64(x), 1e-5, 1e-8, "softmax f32")
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-5)
    # shift invariance (integer shifts are exact in binary32 at this range)
    assert_close(oracle.softmax(x + np.float32(8.0)), y, 1e-5, 1e-9, "shift")
    u = np.full((3, 100), 0.25, np.float32)
    assert np.allclose(oracle.softmax(u), 0.01, rtol=1e-6)
    xh = x.astype(np.float16)
    assert_close(oracle.softmax(xh).astype(np.float64), _softmax64(xh), 1e-3, 1e-4, "softmax f16")


def test_softmax_reference_test_against_torch():
    """test/python/triton/test_softmax.py:75-93: 128x128, torch.rand inputs,
    torch softmax reference, atol 1e-3 (fp16) / 1e-5 (fp32)."""
    torch = pytest.importorskip("torch")
    for dt, atol in ((torch.float16, 1e-3), (torch.float32, 1e-5)):
        x = torch.rand(128, 128, dtype=dt, generator=torch.Generator().manual_seed(0))
        got = torch.from_numpy(oracle.softmax(x.numpy()))
        ref = torch.nn.functional.softmax(x.float(), dim=1).to(dt)
        assert torch.allclose(got, ref, atol=atol)


def test_rmsnorm_vs_float64_and_scale_invariance():
    x = rng(25).normal(0, 2, (32, 4096)).astype(np.float32)
    g = rng(26).normal(1, 0.1, 4096).astype(np.float32)
    x64 = x.astype(np.float64)
    want = x64 / np.sqrt((x64 ** 2).mean(axis=1, keepdims=True) + 1e-6) * g
    y = oracle.rmsnorm(x, g, 1e-6)
    assert_close(y, want, 1e-5, 1e-6, "rmsnorm")
    assert_close(oracle.rmsnorm(x * np.float32(4.0), g, 0.0), oracle.rmsnorm(x, g, 0.0), 1e-5, 1e-6, "scale")
    assert_close(oracle.rmsnorm(x, None, 1e-6), want / g, 1e-5, 1e-6, "no gamma")


def test_rmsnorm_reference_test_against_torch():
    """test/python/triton/test_rms_norm.py:61-86: 127x513, eps 1e-5, torch
    rms_norm reference, atol 1e-2."""
    torch = pytest.importorskip("torch")
    for dt in (torch.float16, torch.float32):
        g = torch.Generator().manual_seed(1)
        x = torch.rand(127, 513, dtype=dt, generator=g)
        w = torch.rand(513, dtype=dt, generator=g)
        got = torch.from_numpy(oracle.rmsnorm(x.numpy(), w.numpy(), 1e-5))
        ref = torch.nn.functional.rms_norm(x.float(), (513,), weight=w.float(), eps=1e-5).to(dt)
        assert torch.allclose(got, ref, atol=1e-2)


def test_layernorm_vs_float64_and_torch():
    """test/python/triton/test_layer_norm.py:84-112: 27x8192 fp32, eps 1e-5,
    torch layer_norm reference, atol 1e-5; mean / rstd as stored at :70-72."""
    torch = pytest.importorskip("torch")
    g = torch.Generator().manual_seed(2)
    x = torch.rand(27, 8192, dtype=torch.float32, generator=g)
    w = torch.rand(8192, dtype=torch.float32, generator=g)
    b = torch.rand(8192, dtype=torch.float32, generator=g)
    y, mean, rstd = oracle.layernorm(x.numpy(), w.numpy(), b.numpy(), 1e-5)
    ref = torch.nn.functional.layer_norm(x, (8192,), weight=w, bias=b, eps=1e-5)
    assert torch.allclose(torch.from_numpy(y), ref, atol=1e-5)
    x64 = x.numpy().astype(np.float64)
    assert_close(mean, x64.mean(axis=1), 2e-5, 1e-7, "mean")  # sequential binary32 sum of 8192
    assert_close(rstd, 1 / np.sqrt(x64.var(axis=1) + 1e-5), 5e-5, 0, "rstd")


def test_silu_mul_vs_float64():
    gv = rng(27).normal(0, 3, (8, 500)).astype(np.float32)
    uv = rng(28).normal(0, 1, (8, 500)).astype(np.float32)
    g64, u64 = gv.astype(np.float64), uv.astype(np.float64)
    assert_close(oracle.silu_mul(gv, uv), g64 / (1 + np.exp(-g64)) * u64, 1e-5, 1e-7, "silu_mul")


# --------------------------------------------------------------------------- #
# Committed fixtures (tests/golden/, written by tests/golden/make_golden.py)
# --------------------------------------------------------------------------- #

def test_golden_fixtures_reproduce():
    meta = json.loads((GOLDEN / "golden.json").read_text())
    data = np.load(GOLDEN / "golden.npz", allow_pickle=False)
    a, b = data["i8_a"], data["i8_b"]
    assert np.array_equal(oracle.gemm_i8_i32(a, b), data["i8_c"])
    assert np.array_equal(oracle.dequant_i32_f16(data["i8_c"], data["i8_sa"], data["i8_sb"]).view(np.uint16),
                          data["i8_c16"])
    assert np.array_equal(oracle.softmax(data["sm_x"]).view(np.uint16), data["sm_y"])
    assert np.array_equal(oracle.rmsnorm(data["rms_x"], data["rms_g"], meta["rms_eps"]).view(np.uint16),
                          data["rms_y"])
    assert meta["seed"] == 20261201


# --------------------------------------------------------------------------- #
# Attention
# --------------------------------------------------------------------------- #

def _sdpa64(q, k, v, scale, causal=False):
    s = np.einsum("bid,bjd->bij", q.astype(np.float64), k.astype(np.float64)) * scale
    if causal:
        nq, nk = s.shape[-2:]
        s = np.where(np.arange(nk)[None, :] > np.arange(nq)[:, None], -np.inf, s)
    s = s - s.max(-1, keepdims=True)
    p = np.exp(s)
    p /= p.sum(-1, keepdims=True)
    return np.einsum("bij,bjd->bid", p, v.astype(np.float64))


@pytest.mark.parametrize("causal", [False, True])
def test_oracle_attention_fp64(causal):
    r = rng(41)
    q = r.uniform(-1, 1, (3, 37, 64)).astype(np.float16)
    k = r.uniform(-1, 1, (3, 53, 64)).astype(np.float16)
    v = r.normal(0, 1, (3, 53, 64)).astype(np.float16)
    got = oracle.attention(q, k, v, 0.3, causal=causal).astype(np.float64)
    want = _sdpa64(q, k, v, 0.3, causal)
    assert np.abs(got - want).max() < 2e-3


def test_oracle_attention_invariants():
    r = rng(42)
    q = r.uniform(0, 1, (2, 40, 64)).astype(np.float16)
    k = r.uniform(0, 1, (2, 70, 64)).astype(np.float16)
    ones = np.ones((2, 70, 64), np.float16)
    assert np.array_equal(oracle.attention(q, k, ones, 0.5), np.ones((2, 40, 64), np.float16))
    v1 = r.normal(0, 1, (2, 1, 64)).astype(np.float16)
    got = oracle.attention(q, k[:, :1], v1, 0.5)
    assert np.array_equal(got, np.broadcast_to(v1, got.shape))
    v = r.normal(0, 1, (2, 70, 64)).astype(np.float16)
    causal = oracle.attention(q, k, v, 0.5, causal=True)
    assert np.array_equal(causal[:, 0], v[:, 0])          # row 0 sees only key 0
    # scale 0: every key weighs the same, whatever the keys are
    uniform = oracle.attention(q, k, v, 0.0)
    assert np.array_equal(uniform, oracle.attention(q, k * 0, v, 0.0))
    assert np.abs(uniform[:, 0].astype(np.float64) - v.astype(np.float64).mean(1)).max() < 1e-3


def test_oracle_attention_matches_torch_at_reference_shape():
    """test/python/triton/test_flash_attention.py: Z = H = 1, N_CTX = 1024,
    D = 64, scale 0.5, torch.rand inputs, rel Frobenius error < 5e-3 against
    scaled_dot_product_attention."""
    import torch
    torch.manual_seed(0)
    q, k, v = (torch.rand(1, 1, 1024, 64) for _ in range(3))
    ref = torch.nn.functional.scaled_dot_product_attention(q, k, v, scale=0.5)
    got = oracle.attention(q.half().numpy(), k.half().numpy(), v.half().numpy(), 0.5)
    rel = float(np.linalg.norm(got.astype(np.float64) - ref.numpy()) / np.linalg.norm(ref.numpy()))
    assert rel < 5e-3, rel


# --------------------------------------------------------------------------- #
# SwiGLU FFN composition
# --------------------------------------------------------------------------- #

def _ffn_float64(x, gamma, eps, wg, sg, wu, su, wd, sd):
    """The block written out in float64 with no intermediate rounding:
    y = (silu(h Wg sg) * (h Wu su)) Wd sd, h = x / sqrt(mean(x^2) + eps) * gamma.
    Shares no code with the oracle (numpy matmuls, no fp16 steps)."""
    x = x.astype(np.float64)
    h = x / np.sqrt((x * x).mean(axis=1, keepdims=True) + eps) * gamma.astype(np.float64)
    g = (h @ wg.astype(np.float64)) * sg.astype(np.float64)
    u = (h @ wu.astype(np.float64)) * su.astype(np.float64)
    a = g / (1.0 + np.exp(-g)) * u
    return (a @ wd.astype(np.float64)) * sd.astype(np.float64)


def _ffn_case(T=48, H=256, I=704, seed=40):
    r = rng(seed)
    wg = r.integers(-127, 128, (H, I), dtype=np.int8)
    wu = r.integers(-127, 128, (H, I), dtype=np.int8)
    wd = r.integers(-127, 128, (I, H), dtype=np.int8)
    sg = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    su = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    sd = (r.uniform(0.5, 1.5, H) / (127 * np.sqrt(I / 3))).astype(np.float16)
    x = r.normal(0, 1, (T, H)).astype(np.float16)
    gamma = r.normal(1, 0.1, H).astype(np.float16)
    return x, gamma, wg, sg, wu, su, wd, sd


def _rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.linalg.norm(got - want) / np.linalg.norm(want))


def test_swiglu_ffn_vs_float64_composition():
    """oracle.swiglu_ffn rounds to fp16 after each of its five stages; the
    float64 composition does not, so they differ by a few fp16 roundings
    (relative 2^-11 each) and nothing more."""
    x, gamma, wg, sg, wu, su, wd, sd = _ffn_case()
    got = oracle.swiglu_ffn(x, gamma, 1e-6, wg, sg, wu, su, wd, sd).astype(np.float64)
    want = _ffn_float64(x, gamma, 1e-6, wg, sg, wu, su, wd, sd)
    assert _rel(got, want) < 2e-3
    assert_close(got, want, 2e-2, 3e-3, "swiglu oracle vs float64")


def test_swiglu_ffn_negative_controls():
    """A swap of the gate and up weights (with their scales), per-channel
    scales applied to the wrong channels (reversed order), a dropped gamma,
    and silu applied to the up branch each move the result far outside the
    bound the oracle meets."""
    x, gamma, wg, sg, wu, su, wd, sd = _ffn_case(seed=41)
    want = _ffn_float64(x, gamma, 1e-6, wg, sg, wu, su, wd, sd)
    bad = {
        "gate/up swapped": oracle.swiglu_ffn(x, gamma, 1e-6, wu, su, wg, sg, wd, sd),
        "down scale on the wrong channels": oracle.swiglu_ffn(x, gamma, 1e-6, wg, sg, wu, su, wd,
                                                              np.ascontiguousarray(sd[::-1])),
        "gate scale on the wrong channels": oracle.swiglu_ffn(x, gamma, 1e-6, wg,
                                                              np.ascontiguousarray(sg[::-1]), wu, su, wd, sd),
        "gamma dropped": oracle.swiglu_ffn(x, np.ones_like(gamma), 1e-6, wg, sg, wu, su, wd, sd),
    }
    for what, y in bad.items():
        assert _rel(y, want) > 5e-2, what
    # silu on the wrong branch, computed from the float64 stages directly
    xf = x.astype(np.float64)
    h = xf / np.sqrt((xf * xf).mean(axis=1, keepdims=True) + 1e-6) * gamma.astype(np.float64)
    g = (h @ wg.astype(np.float64)) * sg.astype(np.float64)
    u = (h @ wu.astype(np.float64)) * su.astype(np.float64)
    wrong = ((u / (1.0 + np.exp(-u)) * g) @ wd.astype(np.float64)) * sd.astype(np.float64)
    got = oracle.swiglu_ffn(x, gamma, 1e-6, wg, sg, wu, su, wd, sd)
    assert _rel(got, wrong) > 5e-2


def test_swiglu_ffn_rows_are_independent():
    """Tokens are independent rows: the block on a row subset equals those
    rows of the block on all rows, bit for bit (what the full-size GPU test
    relies on when it checks sampled token rows)."""
    x, gamma, wg, sg, wu, su, wd, sd = _ffn_case(T=40, seed=42)
    full = oracle.swiglu_ffn(x, gamma, 1e-6, wg, sg, wu, su, wd, sd)
    rows = np.array([0, 7, 39])
    part = oracle.swiglu_ffn(np.ascontiguousarray(x[rows]), gamma, 1e-6, wg, sg, wu, su, wd, sd)
    assert np.array_equal(full[rows].view(np.uint16), part.view(np.uint16))


def test_softmax_relative_gate_catches_a_one_percent_exp_error():
    """The relative gate the C4 softmax GPU test applies (two ulps relative on
    every normal-range fp16 output) accepts a float64 softmax rounded once to
    fp16 and rejects one with a 1% error planted in exp."""
    x16 = rng(12).normal(0, 2, (64, 4096)).astype(np.float16)
    x = x16.astype(np.float64)
    e = np.exp(x - x.max(axis=1, keepdims=True))
    good = (e / e.sum(axis=1, keepdims=True)).astype(np.float16).astype(np.float64)
    # exp 1% high on every other column (a uniform error would cancel in
    # the normalisation)
    e_bad = e * np.where(np.arange(x.shape[1]) % 2 == 0, 1.01, 1.0)
    bad = (e_bad / e_bad.sum(axis=1, keepdims=True)).astype(np.float16).astype(np.float64)
    want = oracle.softmax(x16).astype(np.float64)
    normal = want >= 2.0 ** -14
    ok = lambda y: bool((np.abs(y - want)[normal] <= 2 * 2.0 ** -10 * want[normal]).all())  # noqa: E731
    assert ok(good)
    assert not ok(bad)
