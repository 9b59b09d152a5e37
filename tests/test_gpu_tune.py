"""hx_tune through the C ABI on the GPU: the C2 and C3 (M = 1) shapes tuned
natively, the pinned champions checked against the oracle, a canary fed a
false reference voiding the round (and leaving earlier pins alone), a shape
the family refuses, and the canary reference surviving a pins save/load."""
import numpy as np
import pytest

from conftest import assert_close, rng, to_dev, to_np

import oracle

pytestmark = pytest.mark.gpu

FAST = dict(reps=3, budget_us=20_000.0, min_iters=5, max_iters=40)


def _clear(hx, op, m, n, k):
    hx.config_select(op, m, n, k, -1)


def test_tune_c2_int8_and_pinned_champion_is_exact(hx, dev):
    M = N = K = 4096
    try:
        r = hx.search.tune(1, M, N, K, canary_reference_us=-1.0, **FAST)
        assert r["round_valid"] and r["canary"]["status"] == "baseline", r["canary"]
        timed = [e for e in r["entries"] if e["status"] == "timed"]
        assert len(timed) >= 3, r["entries"]
        assert all(e["status"] in ("timed", "refused") for e in r["entries"]), r["entries"]
        assert r["champion_index"] >= 0 and r["pinned"]
        assert hx.config_lookup(1, M, N, K) == r["champion_index"]
        # the pinned champion on seeded data: sampled rows bit-exact
        a = rng(90).integers(-127, 128, (M, K), dtype=np.int8)
        bt = rng(91).integers(-127, 128, (N, K), dtype=np.int8)
        sa = rng(92).uniform(0.001, 0.02, M).astype(np.float32)
        sb = rng(93).uniform(0.001, 0.02, N).astype(np.float32)
        import torch
        out = torch.empty((M, N), dtype=torch.float16, device=dev)
        c = to_np(hx.gemm_i8(to_dev(a, dev), to_dev(bt, dev), b_layout="nk", row_scale=to_dev(sa, dev),
                             col_scale=to_dev(sb, dev), out=out))
        rows = np.array([0, 777, 2048, 4095])
        want = oracle.dequant_i32_f16(oracle.gemm_i8_i32(a[rows], bt, b_trans=True), sa[rows], sb)
        assert np.array_equal(c[rows].view(np.uint16), want.view(np.uint16))
    finally:
        _clear(hx, 1, M, N, K)


def test_tune_c3_gemv_m1(hx, dev):
    M, N, K = 1, 11008, 4096
    try:
        r = hx.search.tune(6, M, N, K, canary_reference_us=-1.0, **FAST)
        assert r["round_valid"], r["canary"]
        reasons = {e["cfg"]: e["reason"] for e in r["entries"] if e["status"] == "refused"}
        # row-block configs hold M = 1 too; nothing should be wrong or fail
        assert all(e["status"] in ("timed", "refused") for e in r["entries"]), r["entries"]
        assert r["pinned"] and hx.config_lookup(6, M, N, K) == r["champion_index"], reasons
        w = rng(94).integers(-127, 128, (N, K), dtype=np.int8)
        s = rng(95).uniform(0.001, 0.02, N).astype(np.float16)
        x = rng(96).normal(0, 1, (M, K)).astype(np.float16)
        W = hx.ResidentWeight(to_dev(w, dev), to_dev(s, dev), layout="nk")
        try:
            y = to_np(hx.matmul_resident(to_dev(x, dev), W)).astype(np.float32)
        finally:
            W.release()
        want = oracle.matmul(x, w, b_trans=True, scale_n=s.astype(np.float32)).astype(np.float32)
        assert_close(y, want, 1e-2, 1e-3, "tuned gemv")
    finally:
        _clear(hx, 6, M, N, K)


def test_drifted_canary_voids_the_round_and_keeps_earlier_pins(hx, dev):
    M, N, K = 512, 1024, 2048
    op = 2  # f16 x f16
    try:
        first = hx.search.tune(op, M, N, K, canary_reference_us=-1.0, **FAST)
        assert first["round_valid"]
        measured = first["canary"]["q50_us"]
        assert measured and measured > 0
        # pin some config on purpose, then run a round whose canary is
        # judged against a reference a third of what the device measures
        names = [hx.config_get(op, i)["name"] for i in range(hx.config_count(op))]
        keep = names.index("128x128_w2x2")
        hx.config_select(op, M, N, K, keep)
        drift = hx.search.tune(op, M, N, K, canary_reference_us=measured / 3.0, **FAST)
        assert drift["canary"]["status"] == "drift", drift["canary"]
        assert drift["canary"]["shift"] > drift["canary"]["gate"]
        assert not drift["round_valid"] and not drift["pinned"]
        assert hx.config_lookup(op, M, N, K) == keep, "a void round must leave the earlier pin"
        # against the measured reference the same round is steady
        steady = hx.search.tune(op, M, N, K, canary_reference_us=measured, pin=False, **FAST)
        assert steady["canary"]["status"] in ("steady", "drift")
        assert steady["canary"]["status"] == "steady" or abs(steady["canary"]["shift"]) > steady["canary"]["gate"]
        assert hx.config_lookup(op, M, N, K) == keep, "pin=False must not pin"
    finally:
        _clear(hx, op, M, N, K)


def test_refused_shape_pins_nothing(hx, dev):
    # K = 16 int8 bytes is below one 32-byte MFMA k-step: every
    # configuration is refused, there is no champion
    r = hx.search.tune(1, 112, 112, 16, canary_reference_us=-1.0, **FAST)
    assert all(e["status"] == "refused" and e["reason"] == "shallow-k" for e in r["entries"]), r["entries"]
    assert r["champion_index"] == -1 and not r["pinned"]
    assert hx.config_lookup(1, 112, 112, 16) == r["control_index"]
    # K = 100: the tuner's A rows (stride K) are not whole 16-byte chunks
    r = hx.search.tune(1, 100, 100, 100, canary_reference_us=-1.0, **FAST)
    reasons = [(e["status"], e["reason"]) for e in r["entries"]]
    assert all(x == ("refused", "row-stride") for x in reasons), reasons
    # f16 decode family at 40 rows: the products run the tiled GEMM there
    r = hx.search.tune(7, 40, 2048, 512, canary_reference_us=-1.0, **FAST)
    reasons = {(e["status"], e["reason"]) for e in r["entries"]}
    assert reasons == {("refused", "family-shape")} and not r["pinned"], reasons


def test_canary_reference_survives_pins_round_trip(hx, dev):
    M, N, K = 256, 512, 512
    op = 3  # bf16
    try:
        r = hx.search.tune(op, M, N, K, canary_reference_us=-1.0, **FAST)
        assert r["round_valid"]
        text = hx.config_pins_save()
        line = [ln for ln in text.splitlines() if ln.startswith(f"canary {op} ")]
        assert line, text
        q = float(line[0].split()[2])
        assert q == pytest.approx(r["canary"]["q50_us"], rel=1e-5)
        # a reload with the reference doubled: the next round judges against it
        hx.config_pins_load(text.replace(line[0], f"canary {op} {2 * q:.6g}"))
        again = hx.search.tune(op, M, N, K, canary_reference_us=0.0, pin=False, **FAST)
        assert again["canary"]["reference_us"] == pytest.approx(2 * q, rel=1e-5)
        assert again["canary"]["status"] == "drift" and not again["round_valid"]
    finally:
        _clear(hx, op, M, N, K)
