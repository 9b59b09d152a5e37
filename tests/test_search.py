"""The autotune protocol, pinned on the host with the known answers of the
reference's own contract tests (qcom_hexagon_backend/test/
test_hmx_champion_criterion_contract.py and test_hmx_search_loop_contract.py):
the gate max(3xCV, 15%) with ties to the incumbent, the defended walk, the
canary verdicts, inf on failure, the first-rep correctness gate, and the
calibration box.  Plus the gfx950 legality rules over the compiled configs."""
import math

import pytest

INF = float("inf")


@pytest.fixture(scope="module")
def S(hx):
    return hx.search


def row(cfg, tiles, q50, spread=None):
    if spread is None:
        spread = 0.02 * q50
    return dict(cfg=cfg, tiles=list(tiles), q50_us=q50, q20_us=q50 - spread, q80_us=q50 + spread)


def canary(q50=5000.0, spread=100.0):
    return row("canary", (32, 32, 32), q50, spread)


def test_gate_and_cv(S):
    assert (S.CHAMPION_CV_FACTOR, S.CHAMPION_MARGIN_FLOOR) == (3.0, 0.15)
    assert S.champion_gate(0.0) == 0.15
    assert abs(S.champion_gate(0.05) - 0.15) < 1e-12
    assert abs(S.champion_gate(0.10) - 0.30) < 1e-12
    assert abs(S.champion_gate(1.0) - 3.0) < 1e-12
    assert S.champion_gate(None) == 0.15
    assert S.quantile_spread_cv(980, 1000, 1020) == 0.04
    assert S.quantile_spread_cv(None, 1000, 1020) == 0.0
    assert S.quantile_spread_cv(980, INF, 1020) == 0.0
    assert S.quantile_spread_cv(0, 0, 0) == 0.0


def test_tie_goes_to_incumbent(S):
    rep = S.judge_champion_round([row("ctrl", (32, 32, 32), 1000.0), row("edge", (64, 32, 32), 850.0)],
                                 control="ctrl", canary=canary())
    assert rep["champion"] == "ctrl" and rep["changes"] == []
    assert rep["comparisons"][0]["outcome"] == "kept"


def test_crown_is_defended(S):
    rows = [row("ctrl", (32, 32, 32), 1000.0), row("A", (64, 32, 32), 700.0),
            row("B", (32, 64, 32), 900.0), row("C", (128, 32, 32), 640.0)]
    rep = S.judge_champion_round(rows, control="ctrl", iters=300, canary=canary())
    assert rep["round_verdict"] == S.ROUND_VALID
    assert rep["champion"] == "A" and rep["champion_tiles"] == [64, 32, 32]
    assert [c["challenger"] for c in rep["changes"]] == ["A"]
    t = rep["changes"][0]
    assert t["incumbent"] == "ctrl" and abs(t["delta_pct"] - 30.0) < 1e-9 and abs(t["gate_pct"] - 15.0) < 1e-9
    assert {c["challenger"]: c["outcome"] for c in rep["comparisons"]} == {"B": "kept", "A": "takeover", "C": "kept"}
    assert rep["beats_control"]["significant"] is True and rep["champion_significant"] is True
    assert rep["iters"] == 300
    noisy = [row("ctrl", (32, 32, 32), 1000.0, spread=50.0), row("A", (64, 32, 32), 700.0, spread=35.0)]
    assert abs(S.quantile_spread_cv(950, 1000, 1050) - 0.10) < 1e-12
    rep = S.judge_champion_round(noisy, control="ctrl", canary=canary())
    assert rep["champion"] == "ctrl" and abs(rep["comparisons"][0]["gate_pct"] - 30.0) < 1e-9


def test_no_control_is_not_proven(S):
    rows = [row("x", (32, 32, 32), 900.0), row("y", (64, 32, 32), 500.0)]
    rep = S.judge_champion_round(rows, canary=canary())
    assert rep["champion"] == "y" and rep["beats_control"] is None
    assert rep["champion_significant"] is False and "NOT-PROVEN" in rep["significance_note"]
    dead = rows + [row("ctrl", (128, 128, 128), INF)]
    rep = S.judge_champion_round(dead, control=(128, 128, 128), canary=canary())
    assert rep["control"] is None and rep["beats_control"] is None
    assert "never measured" in rep["walk_note"]


def test_unmeasured_is_per_config(S):
    rows = [row("ctrl", (32, 32, 32), 1000.0), row("dead", (64, 64, 64), INF), row("alive", (128, 32, 32), 700.0)]
    rep = S.judge_champion_round(rows, control="ctrl", canary=canary())
    assert rep["unmeasured"] == ["dead"] and rep["champion"] == "alive"
    assert rep["round_verdict"] == S.ROUND_VALID and rep["champion_significant"] is True
    empty = S.judge_champion_round([row("only", (32, 32, 32), INF)], canary=canary())
    assert empty["champion"] is None and empty["unmeasured"] == ["only"]


def test_canary_verdicts(S):
    rows = [row("ctrl", (32, 32, 32), 1000.0), row("A", (64, 32, 32), 700.0)]
    good = S.judge_champion_round(rows, control="ctrl", canary=canary())
    assert good["canary"]["status"] == S.CANARY_REFERENCE and good["champion_significant"]
    judged = S.judge_champion_round(rows, control="ctrl", canary=canary(), canary_reference=canary())
    assert judged["canary"]["status"] == S.CANARY_OK
    for c in (row("canary", (32, 32, 32), INF), None):
        rep = S.judge_champion_round(rows, control="ctrl", canary=c)
        assert rep["round_verdict"] == S.ROUND_INVALID_CANARY
        assert rep["champion"] == "A" and rep["champion_significant"] is False
        assert rep["beats_control"]["significant"] is False and "void" in rep["significance_note"]
    drift = S.judge_champion_round(rows, control="ctrl", canary=canary(8000.0), canary_reference=canary(5000.0))
    assert drift["canary"]["status"] == S.CANARY_DRIFT and "device state moved" in drift["canary"]["reason"]
    assert S.canary_verdict(canary(3000.0), canary(5000.0))["status"] == S.CANARY_DRIFT
    steady = S.canary_verdict(canary(5400.0), canary(5000.0))
    assert steady["status"] == S.CANARY_OK and abs(steady["delta_pct"] - 8.0) < 1e-9
    assert S.canary_verdict(canary(), row("ref", (32, 32, 32), INF))["status"] == S.CANARY_REFERENCE


def test_bench_inf_rules_and_first_rep_gate(S):
    def boom():
        raise RuntimeError("launch failed")
    assert S.bench(boom) == [INF] * 3
    assert S.bench(lambda: (_ for _ in ()).throw(SystemExit(1))) == [INF] * 3
    assert S.bench(lambda: float("nan")) == [INF] * 3
    assert S.bench(lambda: None) == [INF] * 3
    calls = []

    def launch():
        calls.append(1)
        return 10.0
    assert S.bench(launch, reps=3, verify=lambda: False) == [INF] * 3
    assert len(calls) == 1, "a wrong config costs one launch"

    def bad_verify():
        raise FileNotFoundError
    assert S.bench(launch, verify=bad_verify) == [INF] * 3
    n = {"i": 0}

    def drifting():
        n["i"] += 1
        return 1000.0 * n["i"]
    assert S.bench(drifting, reps=3, verify=lambda: True) == [2000.0, 1400.0, 2600.0]


def test_calibration_box(S):
    assert S.calibration_iters(10.0) == 1000
    assert S.calibration_iters(2_600_000.0) == 5
    assert S.calibration_iters(0.0) == 1000
    assert S.calibration_iters(float("nan")) == 1000


def test_gfx950_legality(S, hx):
    gemv = hx.config_get(6, 0)
    assert S.config_verdict(gemv, 16, 11008, 4096) == S.REASON_OK
    assert S.config_verdict(gemv, 17, 11008, 4096) == S.REASON_FAMILY_SHAPE
    big = hx.config_get(1, 0)  # 256x256
    assert (big["bm"], big["bn"]) == (256, 256)
    assert S.config_verdict(big, 4096, 4096, 4096) == S.REASON_OK
    assert S.config_verdict(big, 64, 4096, 4096) == S.REASON_TILE_EXCEEDS_EXTENT
    assert S.config_verdict(dict(big, lds_bytes=200_000), 4096, 4096, 4096) == S.REASON_LDS_BUDGET
    cands = S.enumerate_configs(1, 4096, 4096, 4096)
    assert [c["tiles"] for c in cands] == sorted(c["tiles"] for c in cands)
    assert all(c["verdict"] == S.REASON_OK for c in cands)
    small = S.enumerate_configs(1, 16, 16, 256)
    assert any(c["verdict"] == S.REASON_TILE_EXCEEDS_EXTENT for c in small)
    assert any(c["verdict"] == S.REASON_OK for c in small)


def test_cache_key_and_roundtrip(S, tmp_path):
    k = S.cache_key("b1", "MI355X", "gfx950", 256, 1, 4096, 4096, 4096)
    assert "b1" in k and "4096x4096x4096" in k
    assert k != S.cache_key("b2", "MI355X", "gfx950", 256, 1, 4096, 4096, 4096)
    c = S.TuneCache(tmp_path / "tune.json")
    c.put(k, {"champion": "x", "champion_index": 2, "round_verdict": S.ROUND_VALID})
    c.save()
    c2 = S.TuneCache(tmp_path / "tune.json")
    assert c2.get(k)["champion_index"] == 2
    assert math.isfinite(S.quantile([3.0, 1.0, 2.0], 0.5))
