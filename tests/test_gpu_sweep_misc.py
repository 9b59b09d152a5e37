"""Seeded sweeps against the CPU oracle for the attention forward, the row
kernels and the resident-weight decode path: random shapes (ragged row
lengths, query and key counts that are not multiples of the blocks, a few
to 64 decode rows), both head dims, causal and not, each operand type."""
import numpy as np
import pytest

from conftest import assert_close, bf16_from_f32, rng, to_dev, to_np
from test_gpu_rows import TOL, make, to_torch, values

import oracle

pytestmark = pytest.mark.gpu


def _attn_case(i):
    r = rng(7000 + i)
    D = int(r.choice([64, 128]))
    Nq = int(r.integers(1, 700))
    causal = bool(r.random() < 0.4)
    # causal cases are square half of the time, else any key count
    Nk = Nq if (causal and r.random() < 0.5) else int(r.integers(1, 700))
    return int(r.integers(1, 3)), int(r.integers(1, 5)), Nq, Nk, D, causal, ["f16", "bf16"][i % 2]


ATTN = [_attn_case(i) for i in range(24)]


@pytest.mark.parametrize("Z,H,Nq,Nk,D,causal,dt", ATTN, ids=["-".join(map(str, c)) for c in ATTN])
def test_attention_sweep(hx, dev, Z, H, Nq, Nk, D, causal, dt):
    import torch
    r = rng(Z * 1000 + H * 100 + Nq + 7 * Nk + D)
    raw = [r.normal(0, 1, s).astype(np.float32) for s in ((Z, H, Nq, D), (Z, H, Nk, D), (Z, H, Nk, D))]
    scale = float(D ** -0.5)
    if dt == "bf16":
        q, k, v = (bf16_from_f32(a) for a in raw)
        dv = [to_dev(a.view(np.int16), dev).view(torch.bfloat16) for a in (q, k, v)]
        got = oracle.bf16_bits_to_f32(to_np(hx.attention(*dv, scale=scale, causal=causal)).view(np.uint16))
        want = oracle.bf16_bits_to_f32(oracle.attention(q, k, v, scale, causal=causal, bf16=True).view(np.uint16))
        tol = 3e-2
    else:
        q, k, v = (a.astype(np.float16) for a in raw)
        got = to_np(hx.attention(*(to_dev(a, dev) for a in (q, k, v)), scale=scale, causal=causal)).astype(np.float32)
        want = oracle.attention(q, k, v, scale, causal=causal).astype(np.float32)
        tol = 1e-2
    assert np.abs(got - want).max() < tol
    assert np.linalg.norm(got - want) <= 1e-2 * max(np.linalg.norm(want), 1e-6)


# longest row the register path holds: 4096 16-byte vectors
MAX_COLS = {"f16": 32768, "bf16": 32768, "f32": 16384}


def _row_case(i):
    r = rng(8000 + i)
    dtype = ["f16", "bf16", "f32"][i % 3]
    return int(r.integers(1, 200)), int(r.integers(1, MAX_COLS[dtype] + 1)), dtype


ROWS = [_row_case(i) for i in range(24)]


@pytest.mark.parametrize("rows,cols,dtype", ROWS, ids=["-".join(map(str, c)) for c in ROWS])
def test_rows_sweep(hx, dev, rows, cols, dtype):
    xh, _ = make(dtype, (rows, cols), seed=rows + cols)
    gh, _ = make(dtype, (cols,), sigma=0.1, mean=1.0, seed=cols)
    rtol, atol = TOL[dtype]
    bf = dtype == "bf16"
    y = hx.softmax(to_torch(xh, dtype, dev))
    assert_close(values(to_np(y), dtype), values(oracle.softmax(xh, bf16=bf), dtype), rtol, atol, "softmax")
    y = hx.rms_norm(to_torch(xh, dtype, dev), to_torch(gh, dtype, dev), eps=1e-6)
    assert_close(values(to_np(y), dtype), values(oracle.rmsnorm(xh, gh, 1e-6, bf16=bf), dtype), rtol, atol,
                 "rmsnorm")


def _dec_case(i):
    r = rng(6000 + i)
    return (int(r.integers(1, 65)), int(r.choice([64, 200, 1000, 4104])), int(r.choice([64, 512, 1040, 4096])),
            ["kn", "nk"][i % 2], bool(r.random() < 0.5))


DEC = [_dec_case(i) for i in range(24)]


@pytest.mark.parametrize("M,N,K,layout,residual", DEC, ids=["-".join(map(str, c)) for c in DEC])
def test_resident_decode_sweep(hx, dev, M, N, K, layout, residual):
    r = rng(M + N + K)
    w = r.integers(-127, 128, (K, N), dtype=np.int8)
    s = r.uniform(0.001, 0.02, N).astype(np.float16)
    x = r.normal(0, 1, (M, K)).astype(np.float16)
    res = r.normal(0, 1, (M, N)).astype(np.float16) if residual else None
    wl = w if layout == "kn" else np.ascontiguousarray(w.T)
    W = hx.ResidentWeight(to_dev(wl, dev), to_dev(s, dev), layout=layout)
    try:
        y = hx.matmul_resident(to_dev(x, dev), W, residual=None if res is None else to_dev(res, dev))
        got = to_np(y).astype(np.float32)
    finally:
        W.release()
    want = oracle.matmul(x, w, scale_n=s.astype(np.float32), residual=res).astype(np.float32)
    assert_close(got, want, 1e-2, 2e-3, f"resident {M}x{N}x{K} {layout}")


@pytest.mark.parametrize("dtype", ["f16", "f32"])
def test_rows_longest_and_beyond(hx, dev, dtype):
    """The longest row the register path holds, and one element more (the
    two-pass streaming path), both against the oracle."""
    n = MAX_COLS[dtype]
    rtol, atol = TOL[dtype]
    for cols, seed in ((n, 5), (n + 1, 6)):
        xh, _ = make(dtype, (2, cols), seed=seed)
        y = hx.softmax(to_torch(xh, dtype, dev))
        assert_close(values(to_np(y), dtype), values(oracle.softmax(xh), dtype), rtol, atol, f"softmax {cols}")
