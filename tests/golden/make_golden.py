"""Writes tests/golden/golden.npz + golden.json: small known-answer vectors
for the hot path, produced by the oracle and cross-checked here against
independent numpy computations before they are saved.

The reference ships no numeric fixtures for these ops (its device tests
draw torch.rand at run time), so these are this build's own frozen vectors:
  i8_*   64x64x64 int8 GEMM (exact int32) + fp32 row/col scales -> fp16
  sm_*   4x256 fp16 softmax, inputs N(0, 2) (standard deviation 2)
  rms_*  4x256 fp16 RMSNorm, gamma N(1, 0.1), eps 1e-6
Run: python tests/golden/make_golden.py
"""
import json
import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
import oracle  # noqa: E402

SEED = 20261201


def main():
    r = np.random.default_rng(SEED)
    a = r.integers(-127, 128, (64, 64), dtype=np.int8)
    b = r.integers(-127, 128, (64, 64), dtype=np.int8)
    sa = r.uniform(0.001, 0.02, 64).astype(np.float32)
    sb = r.uniform(0.001, 0.02, 64).astype(np.float32)
    c = oracle.gemm_i8_i32(a, b)
    assert np.array_equal(c, a.astype(np.int64) @ b.astype(np.int64))
    c16 = oracle.dequant_i32_f16(c, sa, sb)
    assert np.array_equal(c16, ((c.astype(np.float32) * sa[:, None]) * sb[None, :]).astype(np.float16))
    x = r.normal(0, 2, (4, 256)).astype(np.float16)
    y = oracle.softmax(x)
    x64 = x.astype(np.float64)
    e = np.exp(x64 - x64.max(1, keepdims=True))
    assert np.allclose(y.astype(np.float64), e / e.sum(1, keepdims=True), rtol=1e-3, atol=1e-4)
    xr = r.normal(0, 2, (4, 256)).astype(np.float16)
    g = r.normal(1, 0.1, 256).astype(np.float16)
    yr = oracle.rmsnorm(xr, g, 1e-6)
    xr64 = xr.astype(np.float64)
    ref = xr64 / np.sqrt((xr64 ** 2).mean(1, keepdims=True) + 1e-6) * g.astype(np.float64)
    assert np.allclose(yr.astype(np.float64), ref, rtol=1e-3, atol=1e-4)
    np.savez_compressed(HERE / "golden.npz", i8_a=a, i8_b=b, i8_sa=sa, i8_sb=sb, i8_c=c,
                        i8_c16=c16.view(np.uint16), sm_x=x, sm_y=y.view(np.uint16), rms_x=xr,
                        rms_g=g, rms_y=yr.view(np.uint16))
    (HERE / "golden.json").write_text(json.dumps({
        "seed": SEED, "rms_eps": 1e-6,
        "distributions": {"i8": "uniform integers [-127, 127]", "scales": "uniform [0.001, 0.02] fp32",
                          "softmax_x": "normal mean 0, standard deviation 2 (fp16)",
                          "rms_x": "normal mean 0, standard deviation 2 (fp16)",
                          "rms_gamma": "normal mean 1, standard deviation 0.1 (fp16)"},
        "producer": "oracle/hx_oracle.c via tests/golden/make_golden.py"}, indent=1))


if __name__ == "__main__":
    main()
