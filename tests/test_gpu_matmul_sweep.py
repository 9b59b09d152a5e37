"""Seeded sweep of hx_matmul over shapes, operand types, weight layouts,
column scales and residuals, each case against the CPU oracle.  The shapes
cross every dispatch route of the entry point: the decode GEMVs (M <= 16 in
place on [K][N] weights, M <= 64 streaming with row blocks on [N][K]), the
tiled MFMA GEMM with its default config (split-K ones included), the [K][N]
tiled kernel, and the generic kernel for K that is not a whole number of
16-byte chunks.  Tolerances: binary32 accumulation in another order plus one
output rounding (f16: rtol 1e-2, atol 2e-3; bf16: rtol 2e-2, atol 2e-2)."""
import numpy as np
import pytest

from conftest import assert_close, bf16_from_f32, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu

MS = [1, 2, 3, 4, 7, 16, 17, 33, 64, 65, 130, 300, 520]
NS = [8, 24, 64, 200, 520, 1000, 2056]
KS = [16, 64, 104, 200, 512, 1040, 2048, 4100]


def case(i):
    r = rng(9000 + i)
    kind = ["f16", "bf16", "w8"][i % 3]
    M, N, K = (int(r.choice(MS)), int(r.choice(NS)), int(r.choice(KS)))
    layout = "kn" if r.random() < 0.5 else "nk"
    scale = bool(r.random() < 0.5) or kind == "w8"
    residual = bool(r.random() < 0.4)
    return kind, M, N, K, layout, scale, residual


CASES = [case(i) for i in range(120)]


@pytest.mark.parametrize("kind,M,N,K,layout,scale,residual", CASES,
                         ids=["-".join(map(str, c)) for c in CASES])
def test_matmul_sweep(hx, dev, kind, M, N, K, layout, scale, residual):
    import torch
    r = rng(M * 7919 + N * 31 + K)
    bf = kind == "bf16"
    a32 = r.uniform(-1, 1, (M, K)).astype(np.float32)
    a = bf16_from_f32(a32) if bf else a32.astype(np.float16)
    if kind == "w8":
        b_kn = r.integers(-127, 128, (K, N), dtype=np.int8)
        s = r.uniform(0.001, 0.02, N).astype(np.float16)
    else:
        b32 = r.uniform(-1, 1, (K, N)).astype(np.float32)
        b_kn = bf16_from_f32(b32) if bf else b32.astype(np.float16)
        s = r.uniform(0.5, 1.5, N).astype(np.float32) if scale else None
    res32 = r.normal(0, 1, (M, N)).astype(np.float32) if residual else None
    res = None if res32 is None else (bf16_from_f32(res32) if bf else res32.astype(np.float16))

    def dv(x):
        t = to_dev(x.view(np.int16) if bf and x.dtype == np.uint16 else x, dev)
        return t.view(torch.bfloat16) if bf and x.dtype == np.uint16 else t

    b = b_kn if layout == "kn" else np.ascontiguousarray(b_kn.T)
    y = hx.matmul(dv(a), dv(b), b_layout=layout, col_scale=None if s is None else to_dev(s, dev),
                  residual=None if res is None else dv(res))
    got = to_np(y)
    want = oracle.matmul(a, b_kn, scale_n=None if s is None else s.astype(np.float32), residual=res,
                         a_bf16=bf, b_bf16=bf, r_bf16=bf and res is not None, out_bf16=bf)
    if bf:
        g = oracle.bf16_bits_to_f32(got.view(np.uint16))
        w = oracle.bf16_bits_to_f32(want.view(np.uint16))
        assert_close(g, w, 2e-2, 2e-2, f"{kind} {M}x{N}x{K} {layout}")
    else:
        assert_close(got.astype(np.float32), want.astype(np.float32), 1e-2, 2e-3, f"{kind} {M}x{N}x{K} {layout}")
