"""The native autotuner's decision rule (hx_tune_decide, the decision half of
hx_tune), checked on the CPU through the C ABI with hand-computed cases:

* the gate is max(3 CV, 15%), CV = (q80 - q20) / q50 of the noisier of the
  fastest configuration and the untuned default (the protocol constant of
  QHB/backend/hmx_search.py champion_gate, :1280-1289);
* the fastest timed configuration replaces the default only when it is
  faster by more than the gate; a margin equal to the gate keeps the
  default;
* configurations that failed, were refused or were wrong never win;
* with no timed default, the fastest configuration is the champion;
* the canary: no reference sets one (baseline, valid); a shift within its
  own gate is steady (valid); beyond it, drift voids the round; an untimed
  canary voids the round.

A GPU test (tests/test_gpu_tune.py) drives the whole of hx_tune."""
import math

import pytest

INF = float("inf")


@pytest.fixture(scope="module")
def S(hx):
    return hx.search


def e(index, q50, spread=0.0, status=0):
    """An entry with quantiles q50 -/+ spread/2 (CV = spread / q50)."""
    return dict(index=index, q50=q50, q20=None if q50 is None else q50 - spread / 2,
                q80=None if q50 is None else q50 + spread / 2, status=status)


def test_gate_floor_and_cv_factor(S):
    # quiet arms: the gate is its 15% floor
    r = S.decide([e(0, 100.0), e(1, 80.0)], control_index=0, canary=e(0, 5.0))
    assert r["gate"] == pytest.approx(0.15)
    assert r["margin"] == pytest.approx(0.20)
    assert r["champion_index"] == 1 and r["best_index"] == 1
    # a noisy control (CV 0.1) lifts the gate to 30%: a 20% win is not enough
    r = S.decide([e(0, 100.0, spread=10.0), e(1, 80.0)], control_index=0, canary=e(0, 5.0))
    assert r["gate"] == pytest.approx(0.30)
    assert r["champion_index"] == 0 and r["best_index"] == 1
    # the noisier arm sets it: CV of the challenger 0.125 -> gate 0.375
    r = S.decide([e(0, 100.0, spread=1.0), e(1, 80.0, spread=10.0)], control_index=0, canary=e(0, 5.0))
    assert r["gate"] == pytest.approx(0.375)


def test_margin_equal_to_gate_keeps_the_default(S):
    # 85 against 100 is exactly the 15% floor: not more than the gate
    r = S.decide([e(0, 100.0), e(3, 85.0)], control_index=0, canary=e(0, 5.0))
    assert r["margin"] == pytest.approx(0.15)
    assert r["champion_index"] == 0
    r = S.decide([e(0, 100.0), e(3, 84.9)], control_index=0, canary=e(0, 5.0))
    assert r["champion_index"] == 3


def test_fastest_is_compared_not_the_walk_order(S):
    # only the fastest candidate is judged against the default, wherever it
    # sits in the list
    rows = [e(2, 90.0), e(0, 100.0), e(5, 70.0), e(1, 88.0)]
    for order in (rows, rows[::-1]):
        r = S.decide(order, control_index=0, canary=e(0, 5.0))
        assert r["best_index"] == 5 and r["champion_index"] == 5
        assert r["margin"] == pytest.approx(0.30)


def test_failures_never_win(S):
    rows = [e(0, 100.0), e(1, 10.0, status=1), e(2, 5.0, status=2), e(3, 1.0, status=3), e(4, 95.0)]
    r = S.decide(rows, control_index=0, canary=e(0, 5.0))
    assert r["best_index"] == 4
    assert r["champion_index"] == 0  # 5% is inside the gate
    # an infinite (unmeasured) time is not timed either
    r = S.decide([e(0, 100.0), e(1, INF)], control_index=0, canary=e(0, 5.0))
    assert r["best_index"] == 0 and r["champion_index"] == 0


def test_no_timed_control(S):
    # the default failed: the fastest configuration is the only evidence
    r = S.decide([e(0, 100.0, status=2), e(1, 60.0), e(2, 50.0)], control_index=0, canary=e(0, 5.0))
    assert r["champion_index"] == 2 and r["control_q50_us"] is None
    # the default is not among the entries at all (generic kernel)
    r = S.decide([e(1, 60.0), e(2, 50.0)], control_index=-1, canary=e(0, 5.0))
    assert r["champion_index"] == 2
    # nothing timed: no champion
    r = S.decide([e(0, None, status=1), e(1, None, status=1)], control_index=0, canary=e(0, 5.0))
    assert r["champion_index"] == -1 and r["best_index"] == -1


def test_canary_rules(S):
    rows = [e(0, 100.0), e(1, 50.0)]
    # no reference: the round establishes one
    r = S.decide(rows, 0, canary=e(0, 5.0, spread=0.1), canary_reference_us=0.0)
    assert r["canary"]["status"] == "baseline" and r["round_valid"]
    # within the gate (4% shift, quiet canary: gate 15%)
    r = S.decide(rows, 0, canary=e(0, 5.2, spread=0.05), canary_reference_us=5.0)
    assert r["canary"]["status"] == "steady" and r["round_valid"]
    assert r["canary"]["shift"] == pytest.approx(0.04)
    # beyond it, either way
    for q in (6.0, 4.0):
        r = S.decide(rows, 0, canary=e(0, q, spread=0.05), canary_reference_us=5.0)
        assert r["canary"]["status"] == "drift" and not r["round_valid"]
    # a noisy canary (CV 0.2) widens its own gate to 60%: a 20% shift is steady
    r = S.decide(rows, 0, canary=e(0, 6.0, spread=1.2), canary_reference_us=5.0)
    assert r["canary"]["gate"] == pytest.approx(0.6)
    assert r["canary"]["status"] == "steady"
    # untimed canary, or none at all: void
    r = S.decide(rows, 0, canary=e(0, None, status=2), canary_reference_us=5.0)
    assert r["canary"]["status"] == "failed" and not r["round_valid"]
    r = S.decide(rows, 0, canary=None, canary_reference_us=5.0)
    assert r["canary"]["status"] == "failed" and not r["round_valid"]
    # the champion is still reported in a void round (it is not pinned)
    assert r["champion_index"] == 1


def test_cv_of_degenerate_quantiles(S):
    # a single repetition has q20 = q50 = q80: CV 0, gate on its floor
    r = S.decide([dict(index=0, q50=100.0), dict(index=1, q50=80.0)], control_index=0, canary=e(0, 5.0))
    assert r["gate"] == pytest.approx(0.15)
    assert math.isfinite(r["margin"])
