"""Tile autotuning for the gfx950 kernels: the search protocol of
hexagon-mlir's QHB/backend/hmx_search.py, scored by measured device time.

What carries over from the reference, function by function:

* ``bench`` (hexagon_bench, hmx_search.py:1109-1156): reps launches, the
  quantile triple [q50, q20, q80]; ANY failure of a launch (an exception, a
  SystemExit, a missing or NaN time) scores [inf]*3 instead of stopping the
  search; ``verify`` runs after every rep and a False or raising verify scores
  inf on the FIRST rep, so a wrong config costs one launch.
* ``calibration_iters`` (:1159-1177): iterations = clamp(target / per-iter, 5, 1000).
* ``quantile_spread_cv`` / ``champion_gate`` (:1254-1289): CV = (q80-q20)/q50,
  gate = max(3 x CV, 15%), strict comparison (a tie keeps the incumbent).
* ``canary_verdict`` (:1292-1368): a known-healthy config re-measured every
  round; missing / unmeasured / drift void the round; no reference yet
  establishes one.
* ``judge_champion_round`` (:1370-1560): a deterministic walk from the control
  arm in (tiles, label) order; a challenger takes the crown only past the gate
  set by the noisier arm; significance means beating the control arm in a
  valid round.

What is MI355X-specific: the search space is the set of kernel
configurations compiled into libhxmi (block tile, wave grid, LDS stages,
split-K, GEMV column tiles -- ``hx_config_get``) instead of (BM, BN, BK)
Triton constexprs, the legality rules are the gfx950 LDS budget and the
kernel's extent rule, timing is HIP events on the launch stream, and the cache
key is (library build id, device, arch, CU count, family, shape) rather than
hashes of the Hexagon build artefacts (tuning_key_int, :416-452).
"""
from __future__ import annotations

import json
import math
from pathlib import Path
from typing import Callable, Iterable, Mapping, Optional, Sequence

# --------------------------------------------------------------------------- #
# Constants
# --------------------------------------------------------------------------- #

CHAMPION_CV_FACTOR = 3.0
CHAMPION_MARGIN_FLOOR = 0.15

CANARY_MISSING = "missing"
CANARY_UNMEASURED = "unmeasured"
CANARY_DRIFT = "drift"
CANARY_REFERENCE = "reference-established"
CANARY_OK = "ok"

ROUND_VALID = "valid"
ROUND_INVALID_CANARY = "invalid-canary"

REASON_OK = "ok"
REASON_LDS_BUDGET = "lds-budget"
REASON_TILE_EXCEEDS_EXTENT = "tile-exceeds-extent"
REASON_FAMILY_SHAPE = "family-shape"

#: gfx950 LDS per workgroup (160 KiB per CU).
LDS_BUDGET = 160 * 1024
#: The W8A16 GEMV family serves M <= 16 (one MFMA 16-row tile).
GEMV_MAX_ROWS = 16

GATE_FORM = "max(3xCV, 15%)"


# --------------------------------------------------------------------------- #
# Statistics
# --------------------------------------------------------------------------- #

def _is_finite(value) -> bool:
    if value is None:
        return False
    try:
        x = float(value)
    except (TypeError, ValueError):
        return False
    return math.isfinite(x)


def _finite_or_none(value):
    return float(value) if _is_finite(value) else None


def quantile(samples: Sequence[float], q: float) -> float:
    """Linear-interpolated quantile of an unsorted sample list (inf if empty)."""
    if not samples:
        return float("inf")
    s = sorted(float(x) for x in samples)
    if len(s) == 1:
        return s[0]
    pos = (len(s) - 1) * q
    lo = int(pos)
    hi = min(lo + 1, len(s) - 1)
    frac = pos - lo
    return s[lo] * (1.0 - frac) + s[hi] * frac


def calibration_iters(per_iter_us: float, target_us: float = 2_000_000.0, lo: int = 5,
                      hi: int = 1000) -> int:
    """Iterations that time-box one measurement: clamp(target/per_iter, lo, hi).
    An unreadable (zero / negative) per-iteration time is treated as 1 us."""
    per = max(float(per_iter_us), 1.0) if _is_finite(per_iter_us) else 1.0
    return max(lo, min(hi, int(target_us / per)))


def quantile_spread_cv(q20, q50, q80) -> float:
    """(q80 - q20) / q50, or 0.0 when any value is missing / non-finite or
    the median is not positive (which leaves the gate on its floor)."""
    if not all(_is_finite(v) for v in (q20, q50, q80)):
        return 0.0
    med = float(q50)
    if med <= 0.0:
        return 0.0
    return max(0.0, (float(q80) - float(q20)) / med)


def champion_gate(cv) -> float:
    """max(3 x CV, 15%): the fraction a challenger must beat the incumbent by."""
    v = float(cv) if _is_finite(cv) else 0.0
    return max(CHAMPION_CV_FACTOR * abs(v), CHAMPION_MARGIN_FLOOR)


# --------------------------------------------------------------------------- #
# The benchmarker
# --------------------------------------------------------------------------- #

def bench(launch: Callable[[], float], quantiles=(0.5, 0.2, 0.8), *, reps: int = 3,
          verify: Optional[Callable[[], bool]] = None) -> list:
    """Score one config: ``launch()`` runs the measured loop once and returns
    its per-iteration device time (us).  Returns the quantiles over reps, or
    [inf]*len(quantiles) on any failure; verify() is checked after each rep
    and a False / raising verify stops at the first rep."""
    samples = []
    for _ in range(max(1, int(reps))):
        try:
            t = launch()
        except (Exception, SystemExit):  # noqa: BLE001 -- a bad config is inf, not fatal
            return [float("inf")] * len(quantiles)
        if not _is_finite(t):
            return [float("inf")] * len(quantiles)
        if verify is not None:
            try:
                ok = verify()
            except (Exception, SystemExit):  # noqa: BLE001
                return [float("inf")] * len(quantiles)
            if not ok:
                return [float("inf")] * len(quantiles)
        samples.append(float(t))
    return [quantile(samples, q) for q in quantiles]


# --------------------------------------------------------------------------- #
# Canary and champion
# --------------------------------------------------------------------------- #

def _record_q50(record):
    if isinstance(record, Mapping):
        v = record.get("q50_us")
    else:
        v = record
    return float(v) if _is_finite(v) else None


def canary_verdict(metrics, reference=None) -> dict:
    """The per-round sentinel: missing / unmeasured / drift are unhealthy;
    with no healthy reference the canary establishes one."""
    rec = dict(status=CANARY_OK, healthy=True, q50_us=None, cv=0.0, reference_q50_us=None,
               delta_pct=None, gate_pct=None, reason="")
    if metrics is None:
        rec.update(status=CANARY_MISSING, healthy=False,
                   reason="no canary measurement rode with this round; a broken device and "
                          "slow configs cannot be told apart, so no verdict is published")
        return rec
    q50 = _record_q50(metrics)
    cv = (quantile_spread_cv(metrics.get("q20_us"), metrics.get("q50_us"), metrics.get("q80_us"))
          if isinstance(metrics, Mapping) else 0.0)
    rec["cv"] = cv
    rec["q50_us"] = _finite_or_none(q50)
    if q50 is None:
        rec.update(status=CANARY_UNMEASURED, healthy=False,
                   reason="the canary config failed or returned no time: a known-healthy "
                          "config that cannot run indicts the device or the launch path")
        return rec
    ref = _record_q50(reference)
    rec["reference_q50_us"] = _finite_or_none(ref)
    if ref is None or ref <= 0.0:
        rec.update(status=CANARY_REFERENCE,
                   reason="no healthy reference existed, so this run establishes it")
        return rec
    gate = champion_gate(cv)
    delta = (q50 - ref) / ref
    rec["delta_pct"] = 100.0 * delta
    rec["gate_pct"] = 100.0 * gate
    if abs(delta) > gate:
        rec.update(status=CANARY_DRIFT, healthy=False,
                   reason=f"the canary moved {100.0 * delta:+.1f}% from its reference, more "
                          f"than the {100.0 * gate:.1f}% gate: the device state moved and every "
                          "other number in this round was taken under it")
        return rec
    rec["reason"] = (f"the canary stayed within {100.0 * abs(delta):.1f}% of its reference "
                     f"(gate {100.0 * gate:.1f}%)")
    return rec


def judge_champion_round(measurements: Iterable[Mapping], *, control=None, canary=None,
                         canary_reference=None, iters=None) -> dict:
    """Walk the measured configs from the control arm; a challenger takes
    the crown only by beating the incumbent by more than the gate."""
    canary_rec = canary_verdict(canary, canary_reference)
    round_valid = bool(canary_rec["healthy"])
    rows = []
    for m in measurements:
        r = dict(m)
        r["tiles_tuple"] = tuple(r.get("tiles") or ())
        rows.append(r)

    def q50(r):
        return _record_q50(r)

    def cv_of(r):
        return quantile_spread_cv(r.get("q20_us"), r.get("q50_us"), r.get("q80_us"))

    def label(r):
        return str(r.get("cfg", ""))

    def is_control(r):
        if control is None:
            return False
        if str(control) == label(r):
            return True
        return (not isinstance(control, str)) and tuple(control) == r["tiles_tuple"]

    measured = [r for r in rows if q50(r) is not None]
    unmeasured = [label(r) for r in rows if q50(r) is None]
    control_rows = [r for r in measured if is_control(r)]
    control_row = control_rows[0] if control_rows else None
    control_any = [r for r in rows if is_control(r)]
    ordered = sorted(measured, key=lambda r: (r["tiles_tuple"], label(r)))

    comparisons, changes = [], []

    def compare(ch, inc, step):
        cq, iq = q50(ch), q50(inc)
        cv = max(cv_of(ch), cv_of(inc))
        gate = champion_gate(cv)
        delta = (iq - cq) / iq
        rec = dict(step=step, challenger=label(ch), incumbent=label(inc),
                   challenger_q50_us=_finite_or_none(cq), incumbent_q50_us=_finite_or_none(iq),
                   delta_pct=100.0 * delta, cv=cv, gate_pct=100.0 * gate, gate_form=GATE_FORM,
                   outcome="kept")
        if delta > gate:
            rec["outcome"] = "takeover"
            changes.append(dict(rec))
        comparisons.append(rec)
        return rec["outcome"] == "takeover"

    incumbent = None
    if control_row is not None:
        incumbent = control_row
        walk_note = ("the incumbent starts at the control config: the winner is judged "
                     "against it, so it defends the crown first")
    elif control_any:
        walk_note = ("the control config was nominated but never measured (it scored inf), "
                     "so there is no arm to judge a win against")
    elif control is not None:
        walk_note = ("the nominated control is not among this round's measurements, so "
                     "there is no arm to judge a win against")
    else:
        walk_note = ("no control arm was nominated: the incumbent starts at the first "
                     "enumerated candidate, so the walk is deterministic but the starting "
                     "point is nominal")
    if incumbent is None and ordered and not control_any and control is None:
        incumbent = ordered[0]

    if incumbent is not None:
        for step, ch in enumerate([r for r in ordered if r is not incumbent]):
            if compare(ch, incumbent, step):
                incumbent = ch

    champ = incumbent
    beats = None
    if control_row is not None and champ is not None:
        cv = max(cv_of(control_row), cv_of(champ))
        gate = champion_gate(cv)
        if champ is control_row:
            beats = dict(delta_pct=0.0, cv=cv, gate_pct=100.0 * gate, gate_form=GATE_FORM,
                         significant=False,
                         note="the control config kept the crown: no candidate beat it by the gate")
        else:
            delta = (q50(control_row) - q50(champ)) / q50(control_row)
            beats = dict(delta_pct=100.0 * delta, cv=cv, gate_pct=100.0 * gate, gate_form=GATE_FORM,
                         significant=bool(round_valid and delta > gate),
                         note=(f"the champion beat the control config by {100.0 * delta:.1f}%, "
                               + ("more than" if delta > gate else "not more than")
                               + f" the {100.0 * gate:.1f}% gate"))
    significant = bool(round_valid and beats is not None and beats["significant"])
    if not round_valid:
        note = ("the round is void (" + canary_rec["status"] + "): " + canary_rec["reason"]
                + ". The champion below is the walk's survivor, not a verdict.")
    elif beats is None:
        note = ("no control arm produced a measurement, so there is nothing to prove a win "
                "against: the champion is the walk's survivor (NOT-PROVEN, which is not the "
                "same as 'no effect')")
    elif beats["significant"]:
        note = f"the champion beat the control config by more than the gate at iters={iters}"
    else:
        note = (f"the champion did not beat the control config by more than the gate at "
                f"iters={iters}: NOT-PROVEN, which is not the same as 'no effect'")
    return dict(
        kind="hx-search-champion", round_verdict=ROUND_VALID if round_valid else ROUND_INVALID_CANARY,
        iters=iters, gate=dict(form=GATE_FORM, cv_factor=CHAMPION_CV_FACTOR,
                               margin_floor=CHAMPION_MARGIN_FLOOR),
        canary=canary_rec, walk_note=walk_note, measured_configs=len(measured),
        champion=label(champ) if champ is not None else None,
        champion_tiles=list(champ["tiles_tuple"]) if champ is not None else None,
        champion_q50_us=_finite_or_none(q50(champ)) if champ is not None else None,
        control=label(control_row) if control_row is not None else None,
        control_tiles=list(control_row["tiles_tuple"]) if control_row is not None else None,
        beats_control=beats, champion_significant=significant, significance_note=note,
        changes=changes, comparisons=comparisons, unmeasured=unmeasured,
        cvs={label(r): _finite_or_none(cv_of(r)) for r in rows})


# --------------------------------------------------------------------------- #
# Legality over the compiled configurations
# --------------------------------------------------------------------------- #

def config_verdict(cfg: Mapping, m: int, n: int, k: int) -> str:
    """Legality of one compiled config for one (M, N, K), in this order:
    the LDS budget, the family's shape domain, and the extent rule: a block
    tile wider than the extent padded to a power of two (and wider than the
    smallest compiled tile, 64) computes only masked rows -- the counterpart
    of tile_ladder stopping at the padded extent (hmx_search.py:246-266)."""
    if int(cfg.get("lds_bytes", 0)) > LDS_BUDGET:
        return REASON_LDS_BUDGET
    pad = lambda x: max(32, 1 << max(0, (int(x) - 1).bit_length()))  # noqa: E731
    if cfg.get("col_tiles", 0):  # GEMV family
        if m > GEMV_MAX_ROWS:
            return REASON_FAMILY_SHAPE
        if 16 * int(cfg["col_tiles"]) > max(16, pad(n)):
            return REASON_TILE_EXCEEDS_EXTENT
        return REASON_OK
    if int(cfg["bm"]) > max(64, pad(m)) or int(cfg["bn"]) > max(64, pad(n)):
        return REASON_TILE_EXCEEDS_EXTENT
    return REASON_OK


def config_tiles(cfg: Mapping) -> tuple:
    """The ordering key of a config in the champion walk."""
    if cfg.get("col_tiles", 0):
        return (16, 16 * int(cfg["col_tiles"]), int(cfg["split_k"]))
    return (int(cfg["bm"]), int(cfg["bn"]), int(cfg["waves_m"]) * int(cfg["waves_n"]))


def enumerate_configs(op: int, m: int, n: int, k: int, get=None, count=None) -> list:
    """Every compiled config of family ``op`` with its verdict for (m, n, k),
    sorted by tiles then index."""
    if get is None or count is None:
        from . import ops
        get, count = ops.config_get, ops.config_count
    out = []
    for i in range(count(op)):
        cfg = get(op, i)
        out.append(dict(index=i, cfg=cfg, tiles=config_tiles(cfg),
                        verdict=config_verdict(cfg, m, n, k)))
    return sorted(out, key=lambda r: (r["tiles"], r["index"]))


# --------------------------------------------------------------------------- #
# Device timing and the full search
# --------------------------------------------------------------------------- #

def time_launches(fn: Callable[[], None], iters: int, warmup: int = 2) -> float:
    """Mean per-launch device time (us) of ``fn`` over ``iters`` launches,
    HIP events on torch's current stream (the stream the library launches on)."""
    import torch
    for _ in range(warmup):
        fn()
    s = torch.cuda.current_stream()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record(s)
    for _ in range(iters):
        fn()
    e1.record(s)
    e1.synchronize()
    return 1000.0 * e0.elapsed_time(e1) / iters


def tune(op: int, m: int, n: int, k: int, run: Callable[[], None],
         verify: Optional[Callable[[], bool]] = None, *, reps: int = 3,
         target_us: float = 200_000.0, canary_reference=None, pin: bool = True) -> dict:
    """Search the compiled configs of family ``op`` for shape (m, n, k).

    ``run()`` performs one call of the operator (whatever config is pinned);
    ``verify()`` checks the output of the last call.  The control arm is the
    untuned default config; the canary is the default config re-measured
    after the sweep.  The champion is pinned with hx_config_select when the
    round is valid and ``pin`` is set."""
    from . import ops
    default_idx = ops.config_lookup(op, m, n, k)
    cands = enumerate_configs(op, m, n, k)
    measurements = []
    per_iter = max(1.0, time_launches(run, 3, warmup=1))
    iters = calibration_iters(per_iter, target_us=target_us, lo=5, hi=200)
    for c in cands:
        label = c["cfg"]["name"]
        row = dict(cfg=label, tiles=list(c["tiles"]), index=c["index"], verdict=c["verdict"])
        if c["verdict"] != REASON_OK:
            row.update(q50_us=None, q20_us=None, q80_us=None)
            measurements.append(row)
            continue
        ops.config_select(op, m, n, k, c["index"])
        q = bench(lambda: time_launches(run, iters), reps=reps, verify=verify)
        row.update(q50_us=q[0], q20_us=q[1], q80_us=q[2])
        measurements.append(row)
    # canary: the default config once more, after the sweep
    ops.config_select(op, m, n, k, default_idx if default_idx >= 0 else -1)
    cq = bench(lambda: time_launches(run, iters), reps=reps, verify=verify)
    canary = dict(cfg="canary-default", q50_us=cq[0], q20_us=cq[1], q80_us=cq[2])
    control = next((c["cfg"]["name"] for c in cands if c["index"] == default_idx), None)
    report = judge_champion_round(
        [r for r in measurements if r.get("q50_us") is not None or r["verdict"] == REASON_OK],
        control=control, canary=canary, canary_reference=canary_reference, iters=iters)
    champ = next((r for r in measurements if r["cfg"] == report["champion"]), None)
    report["champion_index"] = champ["index"] if champ else None
    report["default_index"] = default_idx
    report["shape"] = [m, n, k]
    report["op"] = op
    report["measurements"] = measurements
    if pin:
        ops.config_select(op, m, n, k,
                          champ["index"] if (champ and report["round_verdict"] == ROUND_VALID)
                          else -1)
    return report


# --------------------------------------------------------------------------- #
# Persistent cache of champions
# --------------------------------------------------------------------------- #

def cache_key(build_id: str, device: str, arch: str, cus: int, op: int, m: int, n: int, k: int) -> str:
    """Every field a timing depends on: a rebuilt library, another device or a
    different shape is a different experiment (a cache miss)."""
    return f"{build_id}|{device}|{arch}|{cus}|op{op}|{m}x{n}x{k}"


class TuneCache:
    """JSON file of champions keyed by ``cache_key``."""

    def __init__(self, path):
        self.path = Path(path)
        self.data = {}
        if self.path.exists():
            self.data = json.loads(self.path.read_text())

    def get(self, key: str):
        return self.data.get(key)

    def put(self, key: str, report: dict) -> None:
        self.data[key] = {k: report.get(k) for k in ("champion", "champion_index", "round_verdict",
                                                     "champion_q50_us", "default_index", "iters")}

    def save(self) -> None:
        self.path.write_text(json.dumps(self.data, indent=1, sort_keys=True))

    def apply(self, key_fields: dict) -> bool:
        """Pin the cached champion for one key; True if a valid one existed."""
        from . import ops
        rec = self.get(cache_key(**key_fields))
        if not rec or rec.get("round_verdict") != ROUND_VALID or rec.get("champion_index") is None:
            return False
        ops.config_select(key_fields["op"], key_fields["m"], key_fields["n"], key_fields["k"],
                          int(rec["champion_index"]))
        return True
