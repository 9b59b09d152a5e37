"""Host surface of the native autotuner (``hx_tune`` / ``hx_tune_decide`` in
libhxmi, ``csrc/hx_tune.cpp``).

The tile search of hexagon-mlir's QHB/backend/hmx_search.py runs inside the
library, so a C or C++ caller of the reference's generated wrapper can tune
exactly as Python does.  This module only converts its report to a dict:

``tune(op, m, n, k, ...)``   time every compiled configuration of family
                             ``op`` at (m, n, k) on synthetic operands, check
                             each one's first launch against the generic
                             kernel, pick the champion, judge the canary,
                             and (if the round is valid and ``pin``) pin it.
``decide(entries, ...)``     the decision rule alone (no device work), for
                             checking it on the CPU.

Pins and canary references persist through ``ops.config_pins_save`` /
``ops.config_pins_load`` (the text format of ``hx_config_pins_save``).
"""
from __future__ import annotations

import ctypes
import math
from typing import Iterable, Mapping, Optional

from . import _abi
from ._abi import TuneEntry, TuneOptions, TuneReport, check, load

#: family codes (include/hx.h HX_OP_*)
OPS = dict(_abi.OP_NAMES)


def _entry_dict(e: TuneEntry) -> dict:
    fin = lambda v: float(v) if math.isfinite(v) else None  # noqa: E731
    return {"index": int(e.index), "status": _abi.TUNE_STATUS.get(int(e.status), str(e.status)),
            "q50_us": fin(e.q50_us), "q20_us": fin(e.q20_us), "q80_us": fin(e.q80_us),
            "reason": e.reason.decode()}


def report_dict(r: TuneReport, names: Optional[Mapping[int, str]] = None) -> dict:
    """The C report as a dict (infinite times become None); ``names`` maps
    configuration indices to names when given."""
    fin = lambda v: float(v) if math.isfinite(v) else None  # noqa: E731
    name = (lambda i: names.get(i) if (names is not None and i is not None and i >= 0) else None)  # noqa: E731
    entries = [_entry_dict(r.entries[i]) for i in range(r.n_entries)]
    if names is not None:
        for e in entries:
            e["cfg"] = names.get(e["index"])
    return {
        "op": int(r.op), "shape": [int(r.m), int(r.n), int(r.k)], "iters": int(r.iters),
        "control_index": int(r.control_index), "control": name(int(r.control_index)),
        "control_q50_us": fin(r.control_q50_us),
        "best_index": int(r.best_index), "best": name(int(r.best_index)), "best_q50_us": fin(r.best_q50_us),
        "champion_index": int(r.champion_index), "champion": name(int(r.champion_index)),
        "margin": float(r.margin), "gate": float(r.gate),
        "canary": {"index": int(r.canary_index), "shape": [int(r.canary_m), int(r.canary_n), int(r.canary_k)],
                   "status": _abi.CANARY_STATUS.get(int(r.canary_status), str(r.canary_status)),
                   "q50_us": fin(r.canary_q50_us), "reference_us": fin(r.canary_reference_us) or None,
                   "shift": float(r.canary_shift), "gate": float(r.canary_gate)},
        "round_valid": bool(r.round_valid), "pinned": bool(r.pinned),
        "entries": entries,
    }


def tune(op: int, m: int, n: int, k: int, *, reps: int = 3, budget_us: float = 0.0, min_iters: int = 0,
         max_iters: int = 0, canary_reference_us: float = 0.0, pin: bool = True, seed: int = 0,
         stream=None) -> dict:
    """Run ``hx_tune`` for family ``op`` at (m, n, k) on ``stream`` (torch's
    current stream when None).  ``budget_us`` = 0 keeps the protocol's 2 s
    per repetition; benches pass a smaller budget.  ``canary_reference_us``:
    > 0 judge the canary against it, 0 against the family's held reference,
    < 0 none."""
    lib = load()
    if stream is None:
        import torch
        stream = torch.cuda.current_stream().cuda_stream
    opt = TuneOptions(reps=reps, min_iters=min_iters, max_iters=max_iters, budget_us=budget_us,
                      canary_reference_us=canary_reference_us, pin=1 if pin else 0, seed=seed)
    rep = TuneReport()
    check(lib.hx_tune(op, m, n, k, ctypes.byref(opt), ctypes.byref(rep), ctypes.c_void_p(stream)), "hx_tune")
    from . import ops
    names = {i: ops.config_get(op, i)["name"] for i in range(ops.config_count(op))}
    return report_dict(rep, names)


def _entry(index: int, q50, q20=None, q80=None, status: int = _abi.TUNE_TIMED) -> TuneEntry:
    inf = float("inf")
    e = TuneEntry()
    e.index = index
    e.status = status
    e.q50_us = inf if q50 is None else float(q50)
    e.q20_us = e.q50_us if q20 is None else float(q20)
    e.q80_us = e.q50_us if q80 is None else float(q80)
    return e


def decide(entries: Iterable[Mapping], control_index: int, canary: Optional[Mapping] = None,
           canary_reference_us: float = 0.0) -> dict:
    """``hx_tune_decide`` over plain dicts: each entry has ``index``, ``q50``
    and optionally ``q20``, ``q80``, ``status`` (an HX_TUNE_* code)."""
    lib = load()
    rows = [_entry(e["index"], e.get("q50"), e.get("q20"), e.get("q80"), e.get("status", _abi.TUNE_TIMED))
            for e in entries]
    arr = (TuneEntry * max(1, len(rows)))(*rows)
    can = None
    if canary is not None:
        can = _entry(canary.get("index", 0), canary.get("q50"), canary.get("q20"), canary.get("q80"),
                     canary.get("status", _abi.TUNE_TIMED))
    rep = TuneReport()
    check(lib.hx_tune_decide(arr, len(rows), control_index, ctypes.byref(can) if can is not None else None,
                             float(canary_reference_us), ctypes.byref(rep)), "hx_tune_decide")
    rep.n_entries = len(rows)
    for i, e in enumerate(rows):
        rep.entries[i] = e
    return report_dict(rep)
