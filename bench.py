#!/usr/bin/env python3
"""Benchmark of the hx hot path on one MI355X.

Headline: int8 GEMM M=N=K=4096, A/B int8 uniform
in [-127, 127], exact int32 accumulation, per-row / per-column fp32 scales
U[0.001, 0.02], dequantised to fp16 in the epilogue.  One step = one call of
hx_gemm_i8 on inputs already resident in HBM (B as the resident K-contiguous
weight image).  value = 2*M*N*K / step time, in TOPS (10^12 int8 ops/s).

Also reported (``secondary``), each against its roofline:
  * the same int8 product with the exact int32 result stored (no dequant);
  * W8A16 decode GEMV, M in {1, 4, 16}, N=11008, K=4096, GB/s,
    rotating over >512 MB of weight copies so the 256 MB MALL cannot serve it;
  * softmax and RMSNorm on fp16 [8192 x 4096], GB/s, rotating
    over 6 input/output sets (768 MB);
  * fp16 GEMM 256^3 latency;
  * SwiGLU FFN tokens=2048, hidden=4096, inter=11008, TFLOP/s;
  * the fused attention forward (the reference test's shape and a multi-head
    one, plain and causal), TFLOP/s.

The CPU baseline is the oracle's restatement of the reference's HVX lowering
(the (i,k,j) int32 loop of ScheduleMatmulForHVX plus the dequant), timed on
this host's cores over a bounded row sample of the same workload.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--only headline]
"""
from __future__ import annotations

import argparse
import ctypes
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "int8/fp16 GEMM TOPS + % MFMA peak; W8A16 GEMV GB/s + % HBM peak"
PEAK_INT8_TOPS = 5000.0      # MI355X dense int8 MFMA, 5.0 POP/s
PEAK_F16_TFLOPS = 2500.0     # dense fp16 MFMA
PEAK_HBM_GBS = 8000.0        # HBM3E


def log(msg: str) -> None:
    print(msg, file=sys.stderr, flush=True)


_SLEEP_CYCLES_PER_MS = None


def _sleep_cycles_per_ms() -> float:
    """Rate of torch.cuda._sleep (a bounded spin kernel) on this device."""
    global _SLEEP_CYCLES_PER_MS
    if _SLEEP_CYCLES_PER_MS is None:
        import torch
        s = torch.cuda.current_stream()
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(10_000)
        a.record(s)
        torch.cuda._sleep(5_000_000)
        b.record(s)
        torch.cuda.synchronize()
        _SLEEP_CYCLES_PER_MS = 5_000_000 / max(a.elapsed_time(b), 1e-3)
    return _SLEEP_CYCLES_PER_MS


class Timed(tuple):
    """(ms per launch, whether the queue stayed ahead of the device), the
    median over timed regions, with the per-region figures kept for the
    spread."""

    def __new__(cls, ms, fed, region_ms, launches):
        t = super().__new__(cls, (ms, fed))
        t.region_ms, t.launches = list(region_ms), launches
        return t

    @property
    def ms(self):
        return self[0]

    def spread(self) -> dict:
        """q20 / q50 / q80 of the per-region mean launch time, in us."""
        import numpy as np
        r = np.asarray(self.region_ms) * 1e3
        return {"q20_us": round(float(np.quantile(r, 0.2)), 3), "q50_us": round(float(np.quantile(r, 0.5)), 3),
                "q80_us": round(float(np.quantile(r, 0.8)), 3), "regions": len(r),
                "launches_per_region": self.launches}


#: timed regions behind every figure: the median is reported, q20 / q80
#: beside it (the reference's bench returns [q50, q20, q80] per config,
#: QHB/backend/hmx_search.py:1109-1156)
REGIONS = 5


def event_timed(calls, iters: int, regions: int = REGIONS) -> Timed:
    """Device time per launch of ``iters`` calls (cycling through ``calls``)
    issued back-to-back on the current stream between one HIP event pair on
    that stream, in each of ``regions`` timed regions; the median region is
    the figure.  When the host issues a call in well under the device time
    of one, the queue stays ahead of the device by itself and nothing else
    runs.  Otherwise a bounded spin kernel holds the stream while the host
    queues each region's launches (so host launch cost opens no gaps),
    followed by a few untimed launches that bring the clocks back up."""
    import statistics
    import torch
    s = torch.cuda.current_stream()
    torch.cuda.synchronize()
    n = min(len(calls), 8)
    t = time.perf_counter()
    for c in calls[:n]:
        c()
    host_ms = (time.perf_counter() - t) * 1e3 / n
    torch.cuda.synchronize()
    a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    a.record(s)
    for c in calls[:n]:
        c()
    b.record(s)
    torch.cuda.synchronize()
    dev_ms = a.elapsed_time(b) / n
    hot = max(3, iters // 8)
    spin = host_ms > 0.5 * dev_ms
    hold_ms = 1.0 + 2.0 * host_ms * (iters + hot)
    per, fed = [], True
    for _ in range(regions):
        if spin:
            torch.cuda._sleep(int(hold_ms * _sleep_cycles_per_ms()))
        for i in range(hot):
            calls[i % len(calls)]()
        a.record(s)
        t0 = time.perf_counter()
        for i in range(iters):
            calls[i % len(calls)]()
        queued_ms = (time.perf_counter() - t0) * 1e3
        b.record(s)
        torch.cuda.synchronize()
        ms = a.elapsed_time(b) / iters
        per.append(ms)
        fed = fed and ((queued_ms < hold_ms) if spin else (queued_ms < ms * iters))
    return Timed(statistics.median(per), fed, per, iters)


def clock_during(hx, calls, iters: int) -> dict:
    """The mean shader clock (MHz) of the tiled GEMM workgroups over one
    region of ``iters`` launches (the library's clock probe), or None."""
    try:
        hx.clock_probe(True)
        try:
            for i in range(iters):
                calls[i % len(calls)]()
            r = hx.clock_read()
        finally:
            hx.clock_probe(False)
        return {"mhz": round(r["mhz"], 1), "workgroups": r["workgroups"],
                "method": "s_memtime / s_memrealtime per workgroup (hx_clock_probe), one region of "
                          f"{iters} launches after the timed ones"}
    except Exception as e:  # noqa: BLE001
        return {"mhz": None, "error": str(e)}


PROFILES = ROOT / "profiles"


def traffic_of(kernel_key: str):
    """HBM bytes per launch of one kernel from the committed rocprofv3 --pmc
    summary (profiles/traffic.txt: FETCH_SIZE + WRITE_SIZE, each scaled by
    the same counter's reading on a copy kernel of known size), or None."""
    f = PROFILES / "traffic.txt"
    if not f.exists():
        return None
    for line in f.read_text().splitlines():
        if line.startswith(kernel_key + "="):
            try:
                return int(float(line.split("=", 1)[1].split("#", 1)[0]))
            except ValueError:
                return None
    return None


def roofline(bound, achieved, peak, unit, traffic=None):
    return {"bound": bound, "achieved": round(achieved, 3), "peak": peak, "unit": unit,
            "frac": round(achieved / peak, 4), "traffic": traffic}


# --------------------------------------------------------------------------- #
# Headline: int8 GEMM 4096^3 + dequant
# --------------------------------------------------------------------------- #

#: the native tuner's protocol on the bench path: 3 repetitions of about
#: 50 ms of device time each (the reference's 2 s per repetition would make
#: the default bench run take many minutes)
BENCH_TUNE = dict(reps=3, budget_us=50_000.0, min_iters=5, max_iters=200)


def tune_summary(report):
    """The autotuner's verdict (hx_tune's report), trimmed for the bench line."""
    return {"champion": report.get("champion"), "control": report.get("control"),
            "best": report.get("best"), "margin": round(report.get("margin", 0.0), 4),
            "gate": round(report.get("gate", 0.0), 4), "round_valid": report.get("round_valid"),
            "pinned": report.get("pinned"),
            "canary": {k: report["canary"][k] for k in ("status", "q50_us", "reference_us", "shift")},
            "q50_us": {e["cfg"]: (round(e["q50_us"], 2) if e.get("q50_us") is not None else e["reason"])
                       for e in report.get("entries", [])}}


def tune(hx, op, m, n, k):
    return tune_summary(hx.search.tune(op, m, n, k, **BENCH_TUNE))


def bench_gemm_i8(hx, steps: int, warmup: int, tune_on: bool = True):
    import numpy as np
    import torch
    import oracle
    M = N = K = 4096
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(1234)
    a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    bt = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)  # [N, K]
    sa = torch.empty(M, dtype=torch.float32, device=dev).uniform_(0.001, 0.02, generator=g)
    sb = torch.empty(N, dtype=torch.float32, device=dev).uniform_(0.001, 0.02, generator=g)
    c = torch.empty((M, N), dtype=torch.float16, device=dev)
    step = hx.bind_gemm_i8(a, bt, c, b_layout="nk", row_scale=sa, col_scale=sb)
    tune_report = None
    if tune_on:
        tune_report = tune(hx, 1, M, N, K)
        # a second round: its canary is judged against the reference the
        # first round established, so drift between the two voids it (a
        # fresh process has no reference of its own: pins from another build
        # are refused)
        again = tune(hx, 1, M, N, K)
        tune_report["second_round"] = {"champion": again["champion"], "round_valid": again["round_valid"],
                                       "canary": again["canary"]}

    # a one-row softmax before the warmup and after the timed steps: other
    # hx kernels around them make the headline's launches one phase of a
    # kernel trace (bench.py --stats-from finds it by its length)
    marker_x = torch.zeros((1, 64), dtype=torch.float16, device=dev)
    marker = lambda: hx.softmax(marker_x)  # noqa: E731
    marker()
    hx.manifest_clear()
    hx.manifest_enable(True)
    for _ in range(warmup):
        step()
    hx.manifest_enable(False)
    plan = hx.manifest()["records"]
    # the timed region: K back-to-back steps between one HIP event pair on
    # the launch stream, inside the host-clock bracket (both synchronized)
    s = torch.cuda.current_stream()
    ev_a, ev_b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ev_a.record(s)
    for _ in range(steps):
        step()
    queued_ms = (time.perf_counter() - t0) * 1e3
    ev_b.record(s)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    ev_ms = ev_a.elapsed_time(ev_b) / steps
    fed = queued_ms < ev_ms * steps  # the host stayed ahead of the device
    marker()
    # the spread: more timed regions of the same number of launches (at
    # least 20), and the shader clock the kernel ran at over one more
    spread = event_timed([step], max(steps, 20), regions=7)
    clock = clock_during(hx, [step], max(steps, 20))
    # the same call on all-zero operands (same instructions and accesses, no
    # data switching), timed and clocked the same way right after
    az, bz = torch.zeros_like(a), torch.zeros_like(bt)
    cz = torch.empty_like(c)
    step_z = hx.bind_gemm_i8(az, bz, cz, b_layout="nk", row_scale=sa, col_scale=sb)
    step_z()
    zero_t = event_timed([step_z], max(steps, 20), regions=7)
    zero_clock = clock_during(hx, [step_z], max(steps, 20))
    del az, bz, cz
    ops = 2.0 * M * N * K
    tops_wall = ops / (wall_ms * 1e-3) / 1e12
    tops_kernel = ops / (ev_ms * 1e-3) / 1e12

    # parity spot check on this exact call: sampled rows bit-exact (int32 and fp16)
    rows = np.array([0, 1, 1023, 2048, 4095])
    a_h = a[rows].cpu().numpy()
    bt_h = bt.cpu().numpy()
    acc = oracle.gemm_i8_i32(a_h, bt_h, b_trans=True)
    want = oracle.dequant_i32_f16(acc, sa.cpu().numpy()[rows], sb.cpu().numpy())
    got = c[rows].cpu().numpy()
    exact = bool(np.array_equal(got.view(np.uint16), want.view(np.uint16)))
    cfg_idx = hx.config_lookup(1, M, N, K)
    cfg = hx.config_get(1, cfg_idx)["name"] if cfg_idx >= 0 else "generic"
    return dict(ms_per_step=wall_ms, kernel_ms=ev_ms, tops=tops_wall, tops_kernel=tops_kernel,
                parity_sampled_rows_bitexact=exact, kernel=cfg, inputs=(a, bt, sa, sb), output=c,
                tune=tune_report, queue_fed=fed, plan=plan, spread=spread, clock=clock,
                zero_operands={"us_per_call": round(zero_t[0] * 1e3, 3), "spread": zero_t.spread(),
                               "clock": zero_clock,
                               "note": "the same call on all-zero A and B, right after the spread regions"})


def _host_threads():
    try:
        gomp = ctypes.CDLL("libgomp.so.1")
        return gomp, int(gomp.omp_get_max_threads())
    except OSError:
        return None, os.cpu_count() or 1


def _cpu_model() -> str:
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def _median_time(fn, reps: int) -> float:
    import statistics
    fn()  # warm-up (thread pool, page-in)
    times = []
    for _ in range(reps):
        t = time.perf_counter()
        fn()
        times.append(time.perf_counter() - t)
    return statistics.median(times)


def cpu_baseline_gemm_i8(inputs, march: str, reps: int = 5, gpu_out=None):
    """The oracle's (i,k,j) int32 loop + dequant over the same inputs: one
    warm-up, then the median of ``reps`` runs of the full 4096^3 product on
    all host threads (OpenMP), plus a 256-row sample on one thread.  The
    full product is also compared with the GPU's output, every element."""
    import numpy as np
    import oracle
    a, bt, sa, sb = inputs
    b_kn = np.ascontiguousarray(bt.cpu().numpy().T)   # the reference's linalg [K, N]
    a_h = a.cpu().numpy()
    sa_h, sb_h = sa.cpu().numpy(), sb.cpu().numpy()
    K, N = b_kn.shape
    M = a_h.shape[0]
    last = {}

    def run(rows):
        acc = oracle.gemm_i8_i32(np.ascontiguousarray(a_h[:rows]), b_kn)
        last["out"] = oracle.dequant_i32_f16(acc, sa_h[:rows], sb_h)

    gomp, threads = _host_threads()
    med = _median_time(lambda: run(M), reps)
    full_exact = None
    if gpu_out is not None:
        full_exact = bool(np.array_equal(gpu_out.cpu().numpy().view(np.uint16), last["out"].view(np.uint16)))
    one_core = None
    if gomp is not None:
        gomp.omp_set_num_threads(1)
        try:
            t1 = _median_time(lambda: run(256), 1)
        finally:
            gomp.omp_set_num_threads(threads)
        one_core = round(2.0 * 256 * N * K / t1 / 1e12, 5)
    return {"value": round(2.0 * M * N * K / med / 1e12, 5), "unit": "TOPS", "cores": int(threads),
            "kind": "port",
            "sample": f"full int8 4096^3 GEMM + dequant, oracle/hx_oracle.c hxo_gemm_i8_i32 "
                      f"(i,k,j) loop, median of {reps} runs ({med:.3f} s each) after a warm-up",
            "one_core_value": one_core, "one_core_sample": "256 of 4096 rows on 1 thread",
            "cpu_model": _cpu_model(), "build": f"gcc -O3 -march=native ({march}) -fopenmp",
            "gpu_output_bitexact_all_elements": full_exact}


def _both(gomp, threads, fn_all, fn_one, reps_all=3):
    """Median time of fn_all on every host thread, and of fn_one (usually a
    row sample of the same work) on one thread."""
    t_all = _median_time(fn_all, reps_all)
    t_one = None
    if gomp is not None:
        gomp.omp_set_num_threads(1)
        try:
            t_one = _median_time(fn_one, 1)
        finally:
            gomp.omp_set_num_threads(threads)
    return t_all, t_one


def cpu_baselines_secondary(march: str) -> dict:
    """The oracle's restatement of the reference's linalg path for every
    secondary workload, timed on this host on seeded inputs of the same shape:
    the figure on every host thread (OpenMP: rows, or output columns for the
    few-row products, over the threads) and a one-thread figure beside it,
    each on a stated sample (medians after a warm-up; samples bounded so the
    whole leg stays within about a minute).  Keys match the secondary
    workloads' names."""
    import numpy as np
    import oracle
    gomp, threads = _host_threads()
    r = np.random.default_rng(2024)
    out = {}
    base = {"kind": "port", "cpu_model": _cpu_model(), "build": f"gcc -O3 -march=native ({march}) -fopenmp",
            "cores": threads}

    def entry(value_all, value_one, unit, sample, one_sample, **kw):
        return dict(base, value=value_all, unit=unit, sample=sample, one_core_value=value_one,
                    one_core_sample=one_sample, **kw)

    def gemv_like(key, M, N, K, w, sc):
        x = r.normal(0, 1, (M, K)).astype(np.float16)
        t_all, t_one = _both(gomp, threads, lambda: oracle.matmul(x, w, scale_n=sc, split_cols=True),
                             lambda: oracle.matmul(x, w, scale_n=sc))
        nbytes = N * K + 2 * N + 2 * M * K + 2 * M * N
        out[key] = entry(round(nbytes / t_all / 1e9, 3), round(nbytes / t_one / 1e9, 3) if t_one else None,
                         "GB/s", f"full W8A16 GEMV M={M} N={N} K={K}, hxo_matmul (i,k,j) loop with output "
                                 f"columns over {threads} threads, median of 3 after a warm-up",
                         "the same full product on 1 thread", us_per_call=round(t_all * 1e6, 1))

    # C3: W8A16 decode GEMV
    N, K = 11008, 4096
    w = r.integers(-127, 128, (K, N), dtype=np.int8)
    sc = r.uniform(0.001, 0.02, N).astype(np.float32)
    for M in (1, 4, 16):
        gemv_like(f"gemv_m{M}", M, N, K, w, sc)
    del w
    # the same product at the FFN's down-projection shape, 16 rows
    N, K = 4096, 11008
    w = r.integers(-127, 128, (K, N), dtype=np.int8)
    sc = r.uniform(0.001, 0.02, N).astype(np.float32)
    gemv_like("gemv_down", 16, N, K, w, sc)
    del w
    # C4: softmax / RMSNorm on the full 8192 x 4096 fp16 matrix (1 thread: 512 rows)
    R, C = 8192, 4096
    xr = (r.normal(0, 2, (R, C))).astype(np.float16)
    xs = np.ascontiguousarray(xr[:512])
    gam = r.normal(1, 0.1, C).astype(np.float16)
    for name, fa, fo in (("softmax", lambda: oracle.softmax(xr), lambda: oracle.softmax(xs)),
                         ("rmsnorm", lambda: oracle.rmsnorm(xr, gam, 1e-6), lambda: oracle.rmsnorm(xs, gam, 1e-6))):
        t_all, t_one = _both(gomp, threads, fa, fo)
        g = 2 * C if name == "rmsnorm" else 0
        out[name] = entry(round((2 * R * C * 2 + g) / t_all / 1e9, 3),
                          round((2 * 512 * C * 2 + g) / t_one / 1e9, 3) if t_one else None, "GB/s",
                          f"full {name} fp16 [{R} x {C}], oracle row loop, median of 3 after a warm-up",
                          f"512 of the {R} rows on 1 thread", us_per_call=round(t_all * 1e6, 1))
    del xr, xs
    # vocabulary-length softmax on a 64-row sample of the 2048 x 128256 rows
    R, C = 64, 128256
    xv = (r.normal(0, 2, (R, C))).astype(np.float16)
    xv1 = np.ascontiguousarray(xv[:8])
    t_all, t_one = _both(gomp, threads, lambda: oracle.softmax(xv), lambda: oracle.softmax(xv1))
    out["softmax_vocab"] = entry(round(2 * R * C * 2 / t_all / 1e9, 3),
                                 round(2 * 8 * C * 2 / t_one / 1e9, 3) if t_one else None, "GB/s",
                                 f"softmax fp16 [{R} x {C}] (64 of the 2048 rows), oracle row loop, "
                                 "median of 3 after a warm-up", "8 rows on 1 thread",
                                 us_per_call=round(t_all * 1e6, 1))
    del xv, xv1
    # C1 and the reference's published fp16 matmul shapes (S1, S2, S3)
    for key, (M, N, K) in [("gemm_f16_256", (256, 256, 256))] + [(f"ref_{m}x{n}x{k}", (m, n, k))
                                                                  for (m, n, k) in REF_SHAPES]:
        a = r.uniform(-1, 1, (M, K)).astype(np.float16)
        b = r.uniform(-1, 1, (K, N)).astype(np.float16)
        fn = (lambda a=a, b=b: oracle.matmul(a, b))
        t_all, t_one = _both(gomp, threads, fn, fn, reps_all=5)
        out[key] = entry(round(t_all * 1e6, 2), round(t_one * 1e6, 2) if t_one else None, "us",
                         f"full fp16 {M}x{N}x{K} matmul, hxo_matmul, median of 5 after a warm-up",
                         "the same product on 1 thread", tflops=round(2.0 * M * N * K / t_all / 1e12, 5))
    # fp16 decode at the reference tuner's decode shapes (one row: columns over threads)
    for (M, N, K) in ((1, 8192, 8192), (1, 4096, 16384)):
        x = r.uniform(-1, 1, (M, K)).astype(np.float16)
        wk = r.uniform(-1, 1, (K, N)).astype(np.float16)
        t_all, t_one = _both(gomp, threads, lambda: oracle.matmul(x, wk, split_cols=True),
                             lambda: oracle.matmul(x, wk))
        nbytes = N * K * 2 + 2 * M * K + 2 * M * N
        out[f"dec_{M}x{N}x{K}"] = entry(round(nbytes / t_all / 1e9, 3), round(nbytes / t_one / 1e9, 3) if t_one else None,
                                        "GB/s", f"full fp16 decode {M}x{N}x{K}, hxo_matmul (i,k,j) loop with output "
                                                f"columns over {threads} threads, median of 3 after a warm-up",
                                        "the same full product on 1 thread", us_per_call=round(t_all * 1e6, 1))
        del wk
    # C5: the FFN block on a 64-token sample (tokens are independent rows; 1 thread: 4 tokens)
    T, H, I = 64, 4096, 11008
    wg = r.integers(-127, 128, (H, I), dtype=np.int8)
    wu = r.integers(-127, 128, (H, I), dtype=np.int8)
    wd = r.integers(-127, 128, (I, H), dtype=np.int8)
    sg = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    su = (r.uniform(0.5, 1.5, I) / (127 * np.sqrt(H / 3))).astype(np.float16)
    sd = (r.uniform(0.5, 1.5, H) / (127 * np.sqrt(I / 3))).astype(np.float16)
    xf = r.normal(0, 1, (T, H)).astype(np.float16)
    x4 = np.ascontiguousarray(xf[:4])
    g1 = r.normal(1, 0.1, H).astype(np.float16)
    t_all, t_one = _both(gomp, threads, lambda: oracle.swiglu_ffn(xf, g1, 1e-6, wg, sg, wu, su, wd, sd),
                         lambda: oracle.swiglu_ffn(x4, g1, 1e-6, wg, sg, wu, su, wd, sd), reps_all=1)
    out["ffn"] = entry(round(3 * 2.0 * T * H * I / t_all / 1e12, 5),
                       round(3 * 2.0 * 4 * H * I / t_one / 1e12, 5) if t_one else None, "TFLOP/s",
                       f"{T} of 2048 tokens through the full block (RMSNorm, gate/up/down W8A16 matmuls, "
                       "SiLU*mul), oracle composition, one run after a warm-up", "4 tokens on 1 thread",
                       us_per_call=round(t_all * 1e6, 1))
    del wg, wu, wd
    # attention: the reference test's shape in full, the multi-head shapes on 4 of their 64 heads
    for key, (Z, H, N, D, causal, scale, heads) in (
            ("attn_ref", (1, 1, 1024, 64, False, 0.5, 1)), ("attn_mh", (4, 16, 2048, 128, False, None, 4)),
            ("attn_mh_causal", (4, 16, 2048, 128, True, None, 4))):
        q, k, v = (r.random((heads, N, D)).astype(np.float16) for _ in range(3))
        sc_ = scale if scale is not None else D ** -0.5
        t_all, t_one = _both(gomp, threads, lambda: oracle.attention(q, k, v, sc_, causal),
                             lambda: oracle.attention(q[:1], k[:1], v[:1], sc_, causal), reps_all=1)
        fl = 4.0 * N * N * D * (0.5 if causal else 1.0)
        out[key] = entry(round(heads * fl / t_all / 1e12, 6), round(fl / t_one / 1e12, 6) if t_one else None,
                         "TFLOP/s", f"{heads} of the {Z * H} heads ({N} x {N} x {D}{', causal' if causal else ''}), "
                                    "oracle binary32 softmax(QK^T s)V, one run after a warm-up",
                         "1 head on 1 thread")
    return out


# --------------------------------------------------------------------------- #
# Secondary workloads
# --------------------------------------------------------------------------- #

def bench_gemv(hx, iters: int = 600, tune_on: bool = True, tune_fn=tune):
    import torch
    N, K = 11008, 4096
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(99)
    copies = 12  # 12 x 45 MB = 541 MB > 2x the 256 MB MALL
    res = []
    weights = []
    for _ in range(copies):
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        s = torch.empty(N, dtype=torch.float16, device=dev).uniform_(0.001, 0.02, generator=g)
        weights.append(hx.ResidentWeight(w, s, layout="nk"))
        del w
    try:
        for M in (1, 4, 16):
            x = torch.randn((M, K), dtype=torch.float16, device=dev, generator=g)
            # each weight copy writes its own output, as the layers of a
            # decode step do (back-to-back launches rewriting one buffer pay
            # for its lines moving between the XCDs' L2s: +0.5 us at M = 1,
            # +1.3 us at M = 16)
            ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for _ in weights]
            calls = [hx.bind_matmul_resident(x, w, y) for w, y in zip(weights, ys)]
            for c in calls:
                c()
            tuned = tune_fn(hx, 6, M, N, K) if tune_on else None
            tm = event_timed(calls, iters)
            ev_ms, fed = tm
            nbytes = N * K + 2 * N + 2 * M * K + 2 * M * N
            gbs = nbytes / (ev_ms * 1e-3) / 1e9
            cfg = hx.config_get(6, hx.config_lookup(6, M, N, K))["name"]
            res.append({"workload": f"W8A16 GEMV M={M} N={N} K={K}", "value": round(gbs, 1),
                        "unit": "GB/s", "us_per_call": round(ev_ms * 1e3, 3),
                        "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s",
                                             traffic_of(f"gemv_w8a16_m{M}:{cfg}")),
                        "spread": tm.spread(), "bytes_per_call": nbytes, "kernel": cfg, "tune": tuned,
                        "queue_fed": fed,
                        "mall_defeat": f"rotating {copies} resident weight copies (541 MB), "
                                       "each with its own output"})
    finally:
        for w in weights:
            w.release()
    return res


def bench_gemv_down(hx, iters: int = 400):
    """The int8 decode GEMV at 16 rows on the FFN's down-projection shape
    (N = 4096, K = 11008): the untuned default splits K over workgroups; its
    unsplit base config (the same tiles and waves, K in one part) is timed
    beside it on the same weights."""
    import torch
    M, N, K = 16, 4096, 11008
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(98)
    copies = 12  # 12 x 45 MB > 2x the MALL
    weights = []
    for _ in range(copies):
        w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        sc = torch.empty(N, dtype=torch.float16, device=dev).uniform_(0.001, 0.02, generator=g)
        weights.append(hx.ResidentWeight(w, sc, layout="nk"))
        del w
    try:
        x = torch.randn((M, K), dtype=torch.float16, device=dev, generator=g)
        ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for _ in weights]
        names = [hx.config_get(6, i)["name"] for i in range(hx.config_count(6))]
        hx.config_select(6, M, N, K, -1)
        cfg = hx.config_get(6, hx.config_lookup(6, M, N, K))["name"]
        # the split config's own base: the same tiles per workgroup and waves
        # over K with K in one part (packed_ctC_kwW_sP[_e] -> packed_ctC_kwW)
        import re
        base = re.sub(r"_s\d+(_e)?$", "", cfg)
        if base not in names:
            base = cfg
        times = {}
        try:
            for name in dict.fromkeys((cfg, base)):
                hx.config_select(6, M, N, K, names.index(name))
                calls = [hx.bind_matmul_resident(x, w, y) for w, y in zip(weights, ys)]
                for c in calls:
                    c()
                times[name] = event_timed(calls, iters)
        finally:
            hx.config_select(6, M, N, K, -1)
        tm = times[cfg]
        ev_ms, fed = tm
        nbytes = N * K + 2 * N + 2 * M * K + 2 * M * N
        gbs = nbytes / (ev_ms * 1e-3) / 1e9
        return [{"workload": f"W8A16 GEMV M={M} N={N} K={K} (the FFN's down projection at 16 tokens)",
                 "value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(ev_ms * 1e3, 3),
                 "spread": tm.spread(),
                 "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", None),
                 "bytes_per_call": nbytes, "kernel": cfg, "split_k": hx.config_get(6, names.index(cfg))["split_k"],
                 "unsplit_base": base, "unsplit_base_us_same_weights": round(times[base][0] * 1e3, 3),
                 "queue_fed": fed, "mall_defeat": f"rotating {copies} resident weight copies (541 MB)"}]
    finally:
        for w in weights:
            w.release()


def bench_rows(hx, iters: int = 60):
    import torch
    R, C = 8192, 4096
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(7)
    sets = 6  # 6 x (64 MiB in + 64 MiB out) = 768 MiB
    xs = [(torch.randn((R, C), dtype=torch.float16, device=dev, generator=g) * 2.0) for _ in range(sets)]
    ys = [torch.empty((R, C), dtype=torch.float16, device=dev) for _ in range(sets)]
    gamma = (torch.randn(C, dtype=torch.float16, device=dev, generator=g) * 0.1 + 1.0)
    out = []
    nbytes = 2 * R * C * 2
    for name in ("softmax", "rmsnorm"):
        calls = [hx.bind_row_op(name, xs[i], ys[i], weight=gamma if name == "rmsnorm" else None)
                 for i in range(sets)]
        for c in calls:
            c()
        # one untimed region first: the first regions over freshly allocated
        # sets read 1-2 us slower (25.6 against 23.6 us for softmax when
        # timed first, the same op timed again in the process afterwards)
        event_timed(calls, iters, regions=1)
        tm = event_timed(calls, iters)
        ev_ms, fed = tm
        gbs = (nbytes + (2 * C if name == "rmsnorm" else 0)) / (ev_ms * 1e-3) / 1e9
        out.append({"workload": f"{name} fp16 [{R} x {C}]", "value": round(gbs, 1), "unit": "GB/s",
                    "us_per_call": round(ev_ms * 1e3, 3), "spread": tm.spread(),
                    "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", traffic_of(f"{name}_f16_8192x4096")),
                    "mall_defeat": "rotating 6 input/output sets (768 MiB)", "queue_fed": fed})
    return out


def bench_rows_long(hx, iters: int = 20):
    """Softmax over vocabulary-length rows (2048 x 128256 fp16: the 8-wave
    single-pass kernel, one row per CU), two rotating input / output sets
    (2.1 GB), torch.softmax on the same tensors beside.  GB/s counts the
    algorithmic bytes (one read, one write)."""
    import torch
    R, C = 2048, 128256
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(8)
    xs = [torch.randn((R, C), dtype=torch.float16, device=dev, generator=g) * 2.0 for _ in range(2)]
    ys = [torch.empty_like(x) for x in xs]
    try:
        calls = [hx.bind_row_op("softmax", x, y) for x, y in zip(xs, ys)]
        for c in calls:
            c()
        tm = event_timed(calls, iters)
        ev_ms, fed = tm
        t_ms, _ = event_timed([(lambda x=x, y=y: torch.softmax(x, dim=-1, out=y)) for x, y in zip(xs, ys)], iters)
    finally:
        del xs, ys
        torch.cuda.empty_cache()
    gbs = 2 * R * C * 2 / (ev_ms * 1e-3) / 1e9
    return {"workload": f"softmax fp16 [{R} x {C}] (vocabulary-length rows)", "value": round(gbs, 1),
            "unit": "GB/s", "us_per_call": round(ev_ms * 1e3, 2),
            "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s", traffic_of(f"softmax_f16_{R}x{C}")),
            "spread": tm.spread(), "torch_us_same_tensors": round(t_ms * 1e3, 2), "queue_fed": fed}


def bench_gemm_i8_i32(hx, inputs, iters: int = 50):
    """The headline product with the exact int32 result stored (C 67 MB, no
    dequant): same operands and tile config as the headline, timed in
    right after the fp16-dequant product over the same regions (both see the
    same clock and thermal state, so the output's cost is their ratio),
    sampled rows checked bit-exact against the oracle."""
    import numpy as np
    import torch
    import oracle
    a, bt, sa, sb = inputs
    M, K = a.shape
    N = bt.shape[0]
    c = torch.empty((M, N), dtype=torch.int32, device=a.device)
    step = hx.bind_gemm_i8(a, bt, c, b_layout="nk")
    step()
    # the fp16-dequant product timed alternately with it, so both see the
    # same clock and thermal state: the output's cost is their ratio
    c16 = torch.empty((M, N), dtype=torch.float16, device=a.device)
    step16 = hx.bind_gemm_i8(a, bt, c16, b_layout="nk", row_scale=sa, col_scale=sb)
    t16 = event_timed([step16], iters)
    tm = event_timed([step], iters)
    ev16_ms, ev_ms, fed = t16[0], tm[0], tm[1]
    clk = clock_during(hx, [step], iters)
    tops = 2.0 * M * N * K / (ev_ms * 1e-3) / 1e12
    rows = np.array([0, 2047, 4095])
    want = oracle.gemm_i8_i32(a[rows].cpu().numpy(), bt.cpu().numpy(), b_trans=True)
    exact = bool(np.array_equal(c[rows].cpu().numpy(), want))
    cfg_idx = hx.config_lookup(1, M, N, K)
    return {"workload": f"int8 GEMM M=N=K={M}, exact int32 output (no dequant)",
            "value": round(tops, 1), "unit": "TOPS", "us_per_call": round(ev_ms * 1e3, 3),
            "kernel": hx.config_get(1, cfg_idx)["name"] if cfg_idx >= 0 else "generic",
            "roofline": roofline("mfma", tops, PEAK_INT8_TOPS, "TFLOP/s"),
            "spread": tm.spread(), "clock": clk,
            "f16_dequant_us_same_phase": round(ev16_ms * 1e3, 3),
            "i32_over_f16": round(ev_ms / ev16_ms, 4),
            "parity": {"int32_sampled_rows_bitexact": exact}, "queue_fed": fed}


def bench_gemm_i8_kn(hx, inputs, iters: int = 50):
    """The headline product with B given in the linalg [K][N] orientation
    (N contiguous), fp16 dequant output, the same pinned config as the
    headline; B is read in place by transposing LDS reads (the plan is
    reported), and the M = 2048 half of the product is timed as well.
    Sampled rows checked bit-exact against the oracle."""
    import numpy as np
    import torch
    import oracle
    a, bt, sa, sb = inputs
    M, K = a.shape
    N = bt.shape[0]
    b_kn = bt.t().contiguous()
    c = torch.empty((M, N), dtype=torch.float16, device=a.device)
    step = hx.bind_gemm_i8(a, b_kn, c, b_layout="kn", row_scale=sa, col_scale=sb)
    hx.manifest_clear()
    hx.manifest_enable(True)
    step()
    hx.manifest_enable(False)
    plan = hx.manifest()["records"]
    tm = event_timed([step], iters)
    ev_ms, fed = tm
    tops = 2.0 * M * N * K / (ev_ms * 1e-3) / 1e12
    rows = np.array([0, 2047, 4095])
    acc = oracle.gemm_i8_i32(a[rows].cpu().numpy(), bt.cpu().numpy(), b_trans=True)
    want = oracle.dequant_i32_f16(acc, sa.cpu().numpy()[rows], sb.cpu().numpy())
    exact = bool(np.array_equal(c[rows].cpu().numpy().view(np.uint16), want.view(np.uint16)))
    # the first 2048 rows
    half = M // 2
    c2 = torch.empty((half, N), dtype=torch.float16, device=a.device)
    step2 = hx.bind_gemm_i8(a[:half], b_kn, c2, b_layout="kn", row_scale=sa[:half], col_scale=sb)
    hx.manifest_clear()
    hx.manifest_enable(True)
    step2()
    hx.manifest_enable(False)
    plan2 = hx.manifest()["records"]
    ev2_ms, _ = event_timed([step2], iters)
    exact2 = bool(np.array_equal(c2[rows[:2]].cpu().numpy().view(np.uint16), want[:2].view(np.uint16)))
    del b_kn
    return {"workload": f"int8 GEMM M=N=K={M} + dequant, B as [K][N]",
            "value": round(tops, 1), "unit": "TOPS", "us_per_call": round(ev_ms * 1e3, 3),
            "kernel": plan[0]["config"] if plan else None, "weight": plan[0]["weight"] if plan else None,
            "spread": tm.spread(),
            "roofline": roofline("mfma", tops, PEAK_INT8_TOPS, "TFLOP/s"),
            "m2048": {"us_per_call": round(ev2_ms * 1e3, 3),
                               "TOPS": round(2.0 * half * N * K / (ev2_ms * 1e-3) / 1e12, 1),
                               "weight": plan2[0]["weight"] if plan2 else None,
                               "kernel": plan2[0]["config"] if plan2 else None},
            "parity": {"f16_sampled_rows_bitexact": exact and exact2}, "queue_fed": fed}


def bench_vendor_gemms(hx, inputs, iters: int = 30):
    """The vendor library beside the hand-written kernels on the same
    devices and operands: torch._int_mm (hipBLASLt int8 -> int32) against
    hx_gemm_i8 with the int32 output at 4096^3, and torch.mm (hipBLASLt fp16)
    against hx_matmul at fp16 4096^3 (B as [N][K] for both).  Each pair is
    timed alternately, one region of ``iters`` launches each per round over
    REGIONS rounds, so both see the same clock and thermal state; the
    figures are the medians over the rounds."""
    import statistics
    import torch
    a, bt, sa, sb = inputs
    M, K = a.shape
    N = bt.shape[0]
    out = {"workload": "vendor GEMMs beside hx at 4096^3 (hipBLASLt through torch)", "unit": "us",
           "timing": f"alternating regions of {iters} launches, median of {REGIONS} rounds"}

    def alternate(fa, fb):
        ta, tb = [], []
        for _ in range(REGIONS):
            ta.append(event_timed([fa], iters, regions=1)[0] * 1e3)
            tb.append(event_timed([fb], iters, regions=1)[0] * 1e3)
        return round(statistics.median(ta), 3), round(statistics.median(tb), 3)

    c32 = torch.empty((M, N), dtype=torch.int32, device=a.device)
    hx_call = hx.bind_gemm_i8(a, bt, c32, b_layout="nk")
    try:
        btt = bt.t()  # [K, N] view of the [N, K] weight: the column-major B hipBLASLt takes
        hx_call()
        ref = torch._int_mm(a, btt)
        out["int_mm_equal_to_hx"] = bool(torch.equal(ref, c32))
        out["hx_gemm_i8_i32_us"], out["torch_int_mm_i32_us"] = alternate(hx_call, lambda: torch._int_mm(a, btt))
    except Exception as e:  # noqa: BLE001
        out["hx_gemm_i8_i32_us"] = round(event_timed([hx_call], iters)[0] * 1e3, 3)
        out["torch_int_mm_i32_us"] = None
        out["torch_int_mm_error"] = str(e)[:200]
    g = torch.Generator(device=a.device).manual_seed(21)
    x = torch.empty((M, K), dtype=torch.float16, device=a.device).uniform_(-1, 1, generator=g)
    w = torch.empty((N, K), dtype=torch.float16, device=a.device).uniform_(-1, 1, generator=g)
    y = torch.empty((M, N), dtype=torch.float16, device=a.device)
    y2 = torch.empty_like(y)
    f_hx = hx.bind_matmul(x, w, y, b_layout="nk")
    f_hx()
    out["hx_matmul_f16_us"], out["torch_mm_f16_us"] = alternate(f_hx, lambda: torch.mm(x, w.t(), out=y2))
    out["value"] = out["hx_gemm_i8_i32_us"]
    del x, w, y, y2, c32
    return out


def bench_gemm_f16_small(hx, iters: int = 200):
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(5)
    a = torch.empty((256, 256), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
    b = torch.empty((256, 256), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
    c = torch.empty((256, 256), dtype=torch.float16, device=dev)
    call = lambda: hx.matmul(a, b, b_layout="nk", out=c)  # noqa: E731
    call()
    tm = event_timed([call], iters)
    ev_ms = tm[0]
    tf = 2 * 256 ** 3 / (ev_ms * 1e-3) / 1e12
    return {"workload": "fp16 GEMM 256^3 (configs[0], latency-bound plumbing case)",
            "value": round(ev_ms * 1e3, 3), "unit": "us", "tflops": round(tf, 2), "spread": tm.spread(),
            "roofline": roofline("mfma", tf, PEAK_F16_TFLOPS, "TFLOP/s")}


#: the fp16 matmul shapes the reference publishes timings for (M, N, K;
#: ROADMAP.md:98-100, M, N, K = 1024, 512, 64 in QHB/test/
#: test_hmx_vector_readout_object_gate.py:94), with its frozen-build
#: zero-knob medians on a Hexagon v79 NPU (us)
REF_SHAPES = [(1024, 512, 64), (256, 64, 2048), (128, 128, 128)]
REF_PUBLISHED_US = {(1024, 512, 64): 37.0, (256, 64, 2048): 32.0, (128, 128, 128): 3.0}


def bench_reference_shapes(hx, iters: int = 200):
    """fp16 C = A.B at the three shapes the reference publishes timings for
    (A, B uniform [-1, 1], B in linalg [K][N], fp16 out), beside its numbers.
    Different hardware (a phone NPU): context, not a baseline ratio."""
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(6)
    res = []
    for (M, N, K) in REF_SHAPES:
        a = torch.empty((M, K), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
        b = torch.empty((K, N), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
        c = torch.empty((M, N), dtype=torch.float16, device=dev)
        call = lambda a=a, b=b, c=c: hx.matmul(a, b, b_layout="kn", out=c)  # noqa: E731
        hx.manifest_clear()
        hx.manifest_enable(True)
        call()
        hx.manifest_enable(False)
        plan = hx.manifest()["records"]
        tm = event_timed([call], iters)
        ev_ms, fed = tm
        tf = 2.0 * M * N * K / (ev_ms * 1e-3) / 1e12
        res.append({"workload": f"fp16 matmul {M}x{N}x{K} (the reference's published shape)",
                    "value": round(ev_ms * 1e3, 3), "unit": "us", "tflops": round(tf, 3), "spread": tm.spread(),
                    "roofline": roofline("mfma", tf, PEAK_F16_TFLOPS, "TFLOP/s"),
                    "kernel": f"{plan[0]['plan']}:{plan[0]['config']}" if plan else None,
                    "reference_published_us": REF_PUBLISHED_US[(M, N, K)],
                    "reference_hardware": "Hexagon v79 NPU (ROADMAP.md:98-100, frozen build, zero-knob "
                                          "default); not comparable hardware",
                    "queue_fed": fed})
    return res


def bench_f16_decode(hx, iters: int = 300):
    """fp16 decode products at the reference tuner's decode shapes
    (QHB/test/test_hmx_search_loop_contract.py:100-113: (1, 8192, 8192) and
    (1, 4096, 16384)): a registered f16 weight (its packed decode image),
    rotating over copies larger than twice the 256 MB MALL, each copy
    writing its own output; torch (hipBLASLt) on the same weights beside."""
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(12)
    res = []
    for (M, N, K) in ((1, 8192, 8192), (1, 4096, 16384)):
        nbytes = N * K * 2
        copies = max(2, -(-(600 << 20) // nbytes))
        wts = [torch.empty((N, K), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g) for _ in range(copies)]
        rws = [hx.ResidentWeight(w, None, layout="nk") for w in wts]
        try:
            x = torch.randn((M, K), dtype=torch.float16, device=dev, generator=g)
            ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for _ in rws]
            calls = [hx.bind_matmul_resident(x, w, y) for w, y in zip(rws, ys)]
            hx.manifest_clear()
            hx.manifest_enable(True)
            calls[0]()
            hx.manifest_enable(False)
            plan = hx.manifest()["records"]
            tm = event_timed(calls, iters)
            ev_ms, fed = tm
            t_ms, _ = event_timed([(lambda w=w, y=y: torch.matmul(x, w.t(), out=y)) for w, y in zip(wts, ys)], iters)
        finally:
            for w in rws:
                w.release()
        alg = nbytes + 2 * M * K + 2 * M * N
        gbs = alg / (ev_ms * 1e-3) / 1e9
        res.append({"workload": f"fp16 decode {M}x{N}x{K}, registered weight (the reference tuner's decode shape)",
                    "value": round(gbs, 1), "unit": "GB/s", "us_per_call": round(ev_ms * 1e3, 2),
                    "spread": tm.spread(), "roofline": roofline("hbm", gbs, PEAK_HBM_GBS, "GB/s"),
                    "kernel": f"{plan[0]['plan']}:{plan[0]['config']}" if plan else None,
                    "traffic": traffic_of(f"f16_decode_{M}x{N}x{K}:gemv_{plan[0]['config']}") if plan else None,
                    "torch_us_same_weights": round(t_ms * 1e3, 2), "weight_copies": copies, "queue_fed": fed})
        del wts, rws, ys, calls
        torch.cuda.empty_cache()
    return res


def bench_ffn(hx, iters: int = 20, tune_on: bool = True, tune_fn=tune):
    import torch
    T, H, I = 2048, 4096, 11008
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(11)

    def w(k, n):
        wt = torch.randint(-127, 128, (k, n), dtype=torch.int8, device=dev, generator=g)
        s = torch.empty(n, dtype=torch.float16, device=dev).uniform_(0.5, 1.5, generator=g) / (127 * (k / 3) ** 0.5)
        return hx.ResidentWeight(wt, s.half(), layout="kn")

    Wg, Wu, Wd = w(H, I), w(H, I), w(I, H)
    try:
        x = torch.randn((T, H), dtype=torch.float16, device=dev, generator=g)
        gamma = torch.randn(H, dtype=torch.float16, device=dev, generator=g) * 0.1 + 1.0
        y = torch.empty_like(x)
        call = lambda: hx.swiglu_ffn(x, gamma, 1e-6, Wg, Wu, Wd, out=y)  # noqa: E731
        call()
        tuned = None
        if tune_on:
            # gate/up stage (fused SwiGLU epilogue), then the down projection
            tuned = {"swiglu": tune_fn(hx, 5, T, I, H), "down": tune_fn(hx, 4, T, H, I)}
        tm = event_timed([call], iters)
        ev_ms = tm[0]
        clk = clock_during(hx, [call], iters)
        hx.manifest_clear()
        hx.manifest_enable(True)
        call()
        hx.manifest_enable(False)
        plan = [{k: r[k] for k in ("m", "n", "k", "plan", "config", "config_source")}
                for r in hx.manifest()["records"]]
    finally:
        Wg.release(); Wu.release(); Wd.release()
    flops = 3 * 2.0 * T * H * I
    tf = flops / (ev_ms * 1e-3) / 1e12
    return {"workload": f"SwiGLU FFN tokens={T} hidden={H} inter={I}, int8 weights",
            "value": round(tf, 1), "unit": "TFLOP/s", "us_per_call": round(ev_ms * 1e3, 1),
            "spread": tm.spread(), "clock": clk, "plan": plan,
            "roofline": roofline("mfma", tf, PEAK_F16_TFLOPS, "TFLOP/s"), "tune": tuned}


def bench_attention(hx, iters: int = 20):
    """Fused attention forward: the reference test's configuration
    (test/python/triton/test_flash_attention.py: Z=H=1, N=1024, D=64, scale
    0.5) and a multi-head one, plain and causal.  FLOP = 4*Z*H*Nq*Nk*D
    (halved under the causal mask)."""
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(13)
    out = []
    for (Z, H, N, D, causal, scale) in ((1, 1, 1024, 64, False, 0.5), (4, 16, 2048, 128, False, None),
                                        (4, 16, 2048, 128, True, None)):
        q, k, v = (torch.rand((Z, H, N, D), dtype=torch.float16, device=dev, generator=g)
                   for _ in range(3))
        o = torch.empty_like(q)
        call = lambda: hx.attention(q, k, v, scale=scale, causal=causal, out=o)  # noqa: E731
        call()
        tm = event_timed([call], iters)
        ev_ms, fed = tm
        fl = 4.0 * Z * H * N * N * D * (0.5 if causal else 1.0)
        tf = fl / (ev_ms * 1e-3) / 1e12
        out.append({"workload": f"attention Z={Z} H={H} N={N} D={D}{' causal' if causal else ''} fp16",
                    "value": round(tf, 1), "unit": "TFLOP/s", "us_per_call": round(ev_ms * 1e3, 2),
                    "spread": tm.spread(),
                    "roofline": roofline("mfma", tf, PEAK_F16_TFLOPS, "TFLOP/s"), "queue_fed": fed})
    return out


# --------------------------------------------------------------------------- #

def gemv_ab(hx, rounds: int = 5, iters: int = 400) -> str:
    """Interleaved A/B of the decode GEMV configurations that compete for
    the untuned default: int8 at the C3 shapes (N = 11008, K = 4096,
    registered weights rotating over 12 copies, each its own output), at
    the FFN's down projection (N = 4096, K = 11008) and at N = K = 4096
    (whose 12 copies, 192 MB, fit the 256 MB MALL); f16 packed images at the
    reference tuner's decode shapes and their neighbours (one row) and at
    the down projection's shape (copies totalling more than 600 MB).  Every
    round times every candidate once (one region of ``iters`` launches), so
    all of them see the same clock and thermal drift; the table gives the
    median and q20 / q80 over the rounds.  Markdown on stdout."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(77)
    lines = ["# Decode GEMV defaults: interleaved A/B (bench.py --gemv-ab)", "",
             f"Every round times each candidate once ({iters} launches over rotating registered weight copies, "
             f"each with its own output; HIP events); {rounds} rounds; us per launch, median [q20, q80] over the "
             "rounds.  `*` marks the untuned default.", ""]
    xl = ("gemv_packed_ct1_kw16_xl", "gemv_packed_ct1_kw8_xl", "gemv_packed_ct1_kw16_xl_p")
    shapes = [(6, 11008, 4096, (1, 4, 8, 12, 16),
               ("gemv_packed_ct3_kw16", "gemv_packed_ct3_kw16_e", "gemv_packed_ct3_kw8", "gemv_packed_ct4_kw8",
                "gemv_packed_ct1_kw8_xd", "gemv_packed_ct6_kw16_s2")),
              (6, 4096, 11008, (1, 4, 8, 12, 16),
               ("gemv_packed_ct4_kw16_s4", "gemv_packed_ct4_kw16_s4_e", "gemv_packed_ct2_kw16_s2",
                "gemv_packed_ct1_kw16", "gemv_packed_ct1_kw16_e", "gemv_packed_ct1_kw8", "gemv_packed_ct1_kw8_e")),
              (6, 4096, 4096, (1, 4, 8, 16),
               ("gemv_packed_ct1_kw16", "gemv_packed_ct1_kw16_e", "gemv_packed_ct1_kw8", "gemv_packed_ct1_kw8_e",
                "gemv_packed_ct2_kw8", "gemv_packed_ct1_kw8_xd")),
              (7, 8192, 8192, (1,), xl), (7, 4096, 16384, (1,), xl), (7, 4096, 8192, (1,), xl),
              (7, 11008, 4096, (1,), xl), (7, 16384, 4096, (1,), xl),
              (7, 4096, 11008, (8, 12, 16),
               ("gemv_packed_ct2_kw16_s2", "gemv_packed_ct4_kw16_s4_e", "gemv_packed_ct1_kw8", "gemv_packed_ct1_kw8_e")),
              (7, 4096, 4096, (8, 16), ("gemv_packed_ct1_kw8", "gemv_packed_ct1_kw8_e"))]
    for op, N, K, Ms, cands in shapes:
        names = [hx.config_get(op, i)["name"] for i in range(hx.config_count(op))]
        ws = []
        if op == 6:
            for _ in range(12):
                w = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
                sc = torch.empty(N, dtype=torch.float16, device=dev).uniform_(0.001, 0.02, generator=g)
                ws.append(hx.ResidentWeight(w, sc, layout="nk"))
                del w
        else:
            for _ in range(max(2, -(-(600 << 20) // (2 * N * K)))):
                w = torch.empty((N, K), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
                ws.append(hx.ResidentWeight(w, None, layout="nk"))
                del w
        try:
            lines += [f"## {'int8' if op == 6 else 'f16'}, N = {N}, K = {K}", "",
                      "| M | " + " | ".join(c.replace("gemv_packed_", "") for c in cands) + " |",
                      "|---:|" + "---:|" * len(cands)]
            for M in Ms:
                hx.config_select(op, M, N, K, -1)
                default = names[hx.config_lookup(op, M, N, K)]
                x = torch.randn((M, K), dtype=torch.float16, device=dev, generator=g)
                ys = [torch.empty((M, N), dtype=torch.float16, device=dev) for _ in ws]
                t = {c: [] for c in cands}
                try:
                    for _ in range(rounds):
                        for c in cands:
                            hx.config_select(op, M, N, K, names.index(c))
                            calls = [hx.bind_matmul_resident(x, w, y) for w, y in zip(ws, ys)]
                            t[c].append(event_timed(calls, iters, regions=1)[0] * 1e3)
                finally:
                    hx.config_select(op, M, N, K, -1)
                cells = []
                for c in cands:
                    r = np.asarray(t[c])
                    cells.append(f"{np.median(r):.2f} [{np.quantile(r, 0.2):.2f}, {np.quantile(r, 0.8):.2f}]"
                                 + (" *" if c == default else ""))
                lines.append(f"| {M} | " + " | ".join(cells) + " |")
            lines.append("")
        finally:
            for w in ws:
                w.release()
            del ws
            torch.cuda.empty_cache()
    return "\n".join(lines) + "\n"


def ffn_decode_table(hx, iters: int = 200) -> str:
    """The SwiGLU FFN block (H = 4096, I = 11008, int8 weights) at decode and
    small-prefill token counts: each call alternates between two registered
    weight sets (so the weights stream from HBM, 2 x 271 MB), five timed
    regions of ``iters`` calls, with each stage's route and config from the
    plan manifest.  Markdown on stdout."""
    import torch
    H, I = 4096, 11008
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(17)

    def w(k, n):
        wt = torch.randint(-127, 128, (k, n), dtype=torch.int8, device=dev, generator=g)
        s = torch.empty(n, dtype=torch.float16, device=dev).uniform_(0.5, 1.5, generator=g) / (127 * (k / 3) ** 0.5)
        return hx.ResidentWeight(wt, s.half(), layout="kn")

    sets = [(w(H, I), w(H, I), w(I, H)) for _ in range(2)]
    gamma = torch.randn(H, dtype=torch.float16, device=dev, generator=g) * 0.1 + 1.0
    lines = ["# SwiGLU FFN block at decode token counts (bench.py --ffn-decode)", "",
             f"H = {H}, I = {I}, int8 weights with per-channel scales; calls alternate between two registered "
             f"weight sets; five timed regions of {iters} calls (HIP events); us per call, median [q20, q80]; "
             "the route and config of each stage from the plan manifest.", "",
             "| tokens | us per call | weight GB/s | stages |", "|---:|---:|---:|---|"]
    try:
        for T in (1, 4, 8, 12, 16, 17, 24, 32, 33, 48, 64):
            x = torch.randn((T, H), dtype=torch.float16, device=dev, generator=g)
            y = torch.empty_like(x)
            calls = [(lambda ws=ws: hx.swiglu_ffn(x, gamma, 1e-6, *ws, out=y)) for ws in sets]
            for c in calls:
                c()
            hx.manifest_clear()
            hx.manifest_enable(True)
            calls[0]()
            hx.manifest_enable(False)
            stages = "; ".join(f"{r['plan']}:{r['config']}" for r in hx.manifest()["records"])
            tm = event_timed(calls, iters, regions=5)
            sp = tm.spread()
            us = tm[0] * 1e3
            gbs = 3 * H * I / (us * 1e-6) / 1e9
            lines.append(f"| {T} | {us:.2f} [{sp['q20_us']:.2f}, {sp['q80_us']:.2f}] | {gbs:.0f} | {stages} |")
    finally:
        for ws in sets:
            for r in ws:
                r.release()
    return "\n".join(lines) + "\n"


def rows_ab(hx, rounds: int = 5, iters: int = 60) -> str:
    """Interleaved A/B of the row configurations (one row per workgroup
    against the streaming form at 2, 4 and 8 workgroups per CU), pinned
    through hx_config_select, for softmax, RMSNorm and LayerNorm at the C4
    shape and at longer rows: every round times every configuration once
    (one region of ``iters`` launches rotating over input / output sets of
    more than 600 MB, so the MALL cannot serve them); the table gives the
    median and q20 / q80 over the rounds, and checks every configuration's
    output against the one-row form bit for bit.  Markdown on stdout."""
    import numpy as np
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(78)
    fams = {"softmax": 9, "rmsnorm": 10, "layernorm": 11}
    names = [hx.config_get(9, i)["name"] for i in range(hx.config_count(9))]
    code = {torch.float16: 1, torch.bfloat16: 2, torch.float32: 3}
    lines = ["# Row configurations: interleaved A/B (bench.py --rows-ab)", "",
             f"Every round times each configuration once ({iters} launches rotating over input / output sets of "
             f"more than 600 MB; HIP events); {rounds} rounds; us per launch, median [q20, q80] over the rounds.  "
             "`*` marks the untuned default.  Every configuration's output equals the one-row form's bit for bit.",
             "", "| op | dtype | rows x cols | " + " | ".join(names) + " |", "|---|---|---|" + "---:|" * len(names)]
    for R, C, dt in ((8192, 4096, torch.float16), (8192, 4096, torch.bfloat16), (8192, 4096, torch.float32),
                     (2048, 4096, torch.float16), (4096, 8192, torch.float16), (4096, 16384, torch.float16),
                     (4096, 32768, torch.float16)):
        nbytes = R * C * torch.tensor([], dtype=dt).element_size()
        sets = max(2, -(-(600 << 20) // (2 * nbytes)))
        xs = [(torch.randn((R, C), device=dev, generator=g) * 2.0).to(dt) for _ in range(sets)]
        ys = [torch.empty_like(x) for x in xs]
        gam = (torch.randn(C, device=dev, generator=g) * 0.1 + 1.0).to(dt)
        bet = (torch.randn(C, device=dev, generator=g) * 0.1).to(dt)
        try:
            for op, fam in fams.items():
                hx.config_select(fam, R, C, code[dt], -1)
                default = names[hx.config_lookup(fam, R, C, code[dt])]
                calls = [hx.bind_row_op(op, x, y, weight=None if op == "softmax" else gam,
                                        bias=bet if op == "layernorm" else None) for x, y in zip(xs, ys)]
                t = {c: [] for c in names}
                ref = None
                try:
                    for i, c in enumerate(names):
                        hx.config_select(fam, R, C, code[dt], i)
                        calls[0]()
                        torch.cuda.synchronize()
                        out = ys[0].view(torch.uint8).clone()
                        if ref is None:
                            ref = out
                        elif not torch.equal(out, ref):
                            raise RuntimeError(f"rows A/B: {op} {c} differs from {names[0]} at {R}x{C} {dt}")
                    for _ in range(rounds):
                        for i, c in enumerate(names):
                            hx.config_select(fam, R, C, code[dt], i)
                            t[c].append(event_timed(calls, iters, regions=1)[0] * 1e3)
                finally:
                    hx.config_select(fam, R, C, code[dt], -1)
                cells = []
                for c in names:
                    r = np.asarray(t[c])
                    cells.append(f"{np.median(r):.2f} [{np.quantile(r, 0.2):.2f}, {np.quantile(r, 0.8):.2f}]"
                                 + (" *" if c == default else ""))
                lines.append(f"| {op} | {str(dt)[6:]} | {R} x {C} | " + " | ".join(cells) + " |")
        finally:
            del xs, ys
            torch.cuda.empty_cache()
    return "\n".join(lines) + "\n"


def pmc_workload(hx, keys_path=None) -> None:
    """A few launches of every benchmarked kernel -- every compiled config of
    the headline GEMM and of the decode GEMV, so whichever one the tuner
    picks has a reading, the headline with its int32 output, the row ops and
    the FFN block -- plus a plain 64 MiB copy of known size, for the
    ``rocprofv3 --pmc`` runs (FETCH_SIZE, WRITE_SIZE, the MFMA / LDS / clock
    counters; the copy's readings give the scale from counter to bytes).
    The order is the one ``pmc_sequence`` lists."""
    import torch
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(3)
    src = torch.empty(64 << 20, dtype=torch.uint8, device=dev).random_(generator=g)
    dst = torch.empty_like(src)
    for _ in range(3):
        dst.copy_(src)
    M = N = K = 4096
    a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
    bt = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
    sa = torch.rand(M, device=dev) * 0.02
    sb = torch.rand(N, device=dev) * 0.02
    c = torch.empty((M, N), dtype=torch.float16, device=dev)
    for idx in range(hx.config_count(1)):
        hx.config_select(1, M, N, K, idx)
        for _ in range(3):
            hx.gemm_i8(a, bt, b_layout="nk", row_scale=sa, col_scale=sb, out=c)
    hx.config_select(1, M, N, K, -1)
    c32 = torch.empty((M, N), dtype=torch.int32, device=dev)
    for _ in range(3):
        hx.gemm_i8(a, bt, b_layout="nk", out=c32)
    # the headline's config on all-zero operands: the same instructions and
    # accesses, no data switching in the MFMA units
    az, bz = torch.zeros_like(a), torch.zeros_like(bt)
    for _ in range(3):
        hx.gemm_i8(az, bz, b_layout="nk", row_scale=sa, col_scale=sb, out=c)
    del c32, a, bt, c, az, bz
    w = torch.randint(-127, 128, (11008, 4096), dtype=torch.int8, device=dev, generator=g)
    rw = hx.ResidentWeight(w, torch.rand(11008, device=dev).half() * 0.02, layout="nk")
    for m in (1, 4, 16):
        x = torch.randn((m, 4096), dtype=torch.float16, device=dev, generator=g)
        for idx in range(hx.config_count(6)):
            hx.config_select(6, m, 11008, 4096, idx)
            for _ in range(3):
                hx.matmul_resident(x, rw)
        hx.config_select(6, m, 11008, 4096, -1)
    rw.release()
    xr = torch.randn((8192, 4096), dtype=torch.float16, device=dev, generator=g)
    yr = torch.empty_like(xr)
    gam = torch.ones(4096, dtype=torch.float16, device=dev)
    for _ in range(3):
        hx.softmax(xr, out=yr)
    for _ in range(3):
        hx.rms_norm(xr, gam, 1e-6, out=yr)
    del xr, yr
    T, H, I = 2048, 4096, 11008

    def wt(k, n):
        m = torch.randint(-127, 128, (k, n), dtype=torch.int8, device=dev, generator=g)
        s = (torch.rand(n, device=dev) + 0.5) / (127 * (k / 3) ** 0.5)
        return hx.ResidentWeight(m, s.half(), layout="kn")

    Wg, Wu, Wd = wt(H, I), wt(H, I), wt(I, H)
    x = torch.randn((T, H), dtype=torch.float16, device=dev, generator=g)
    y = torch.empty_like(x)
    for _ in range(3):
        hx.swiglu_ffn(x, gam, 1e-6, Wg, Wu, Wd, out=y)
    # the gate/up GEMM on its persistent config
    sw = [hx.config_get(5, i)["name"] for i in range(hx.config_count(5))]
    hx.config_select(5, T, I, H, sw.index("swiglu_256x128_w2x4_p"))
    for _ in range(3):
        hx.swiglu_ffn(x, gam, 1e-6, Wg, Wu, Wd, out=y)
    hx.config_select(5, T, I, H, -1)
    Wg.release(); Wu.release(); Wd.release()
    del x, y
    # fp16 decode on a registered weight (its packed image), then softmax
    # over vocabulary-length rows
    wf = torch.empty((8192, 8192), dtype=torch.float16, device=dev).uniform_(-1, 1, generator=g)
    rf = hx.ResidentWeight(wf, None, layout="nk")
    xf = torch.randn((1, 8192), dtype=torch.float16, device=dev, generator=g)
    for _ in range(3):
        hx.matmul_resident(xf, rf)
    rf.release()
    del wf
    xv = torch.randn((2048, 128256), dtype=torch.float16, device=dev, generator=g)
    yv = torch.empty_like(xv)
    for _ in range(3):
        hx.softmax(xv, out=yv)
    del xv, yv
    torch.cuda.synchronize()
    if keys_path:
        Path(keys_path).write_text(json.dumps(pmc_sequence(hx)))
    print("pmc workload done", flush=True)


#: kernels the counter parsers read, in pmc_workload's launch order
MEASURED_KERNELS = r"void hx::(gemm_kernel|gemm_generic_kernel|gemv_stream_kernel|row_vec_kernel|row_stream_kernel|row_kernel)<"


def pmc_sequence(hx):
    """(key, launches) of the measured kernels in pmc_workload's order; a
    key repeated across an interleaved group (the FFN block's three kernels
    per call) is listed per call."""
    seq = []
    for idx in range(hx.config_count(1)):
        seq.append((f"gemm_i8_4096_dequant_f16:{hx.config_get(1, idx)['name']}", 3))
    head = hx.config_get(1, hx.config_lookup(1, 4096, 4096, 4096))["name"]
    seq.append((f"gemm_i8_4096_i32:{head}", 3))
    seq.append((f"gemm_i8_4096_dequant_f16_zero_operands:{head}", 3))
    for m in (1, 4, 16):
        for idx in range(hx.config_count(6)):
            seq.append((f"gemv_w8a16_m{m}:{hx.config_get(6, idx)['name']}", 3))
    seq += [("softmax_f16_8192x4096", 3), ("rmsnorm_f16_8192x4096", 3)]
    gu = hx.config_get(5, hx.config_lookup(5, 2048, 11008, 4096))["name"]
    dn = hx.config_get(4, hx.config_lookup(4, 2048, 4096, 11008))["name"]
    for _ in range(3):
        seq += [("ffn_rmsnorm_2048x4096", 1), (f"ffn_gate_up:{gu}", 1), (f"ffn_down:{dn}", 1)]
    for _ in range(3):
        seq += [("ffn_rmsnorm_2048x4096", 1), ("ffn_gate_up:swiglu_256x128_w2x4_p", 1), (f"ffn_down:{dn}", 1)]
    fd = hx.config_get(7, hx.config_lookup(7, 1, 8192, 8192))["name"]
    seq += [(f"f16_decode_1x8192x8192:{fd}", 3), ("softmax_f16_2048x128256", 3)]
    return seq


def _per_dispatch(path):
    """{dispatch id: (kernel name, {counter: summed value}, row)} of a
    rocprofv3 counter-collection CSV (values summed over dimensions)."""
    import csv
    rows = {}
    for r in csv.DictReader(open(path)):
        d = int(r["Dispatch_Id"])
        ent = rows.setdefault(d, [r["Kernel_Name"], {}, r])
        ent[1][r["Counter_Name"]] = ent[1].get(r["Counter_Name"], 0.0) + float(r["Counter_Value"])
    return [rows[d] for d in sorted(rows)]


def _group(keys, dispatches):
    """Map the measured dispatches onto the (key, launches) sequence that
    pmc_workload recorded."""
    import re
    measured = re.compile(MEASURED_KERNELS)
    seq = [d for d in dispatches if measured.match(d[0])]
    out, pos = {}, 0
    for key, n in keys:
        vals = seq[pos:pos + n]
        pos += n
        assert len(vals) == n and len({v[0] for v in vals}) == 1, f"{key}: {[v[0][:60] for v in vals]}"
        out.setdefault(key, []).extend(vals)
    assert pos == len(seq), f"{len(seq) - pos} unmatched launches"
    return out


def traffic_from_pmc(fetch_csv: str, write_csv: str, keys_json: str) -> str:
    """Turn the two counter-collection CSVs of ``--pmc-workload`` runs into
    the key=value lines of profiles/traffic.txt (bytes per launch).  Each
    counter is scaled by its reading on the 64 MiB copies (bytes / counter
    value)."""
    import statistics
    fetch, write = _per_dispatch(fetch_csv), _per_dispatch(write_csv)
    assert [k for k, _, _ in fetch] == [k for k, _, _ in write], "the two runs launched different kernels"
    copy = 64 << 20
    cf = [v["FETCH_SIZE"] for k, v, _ in fetch if k == "__amd_rocclr_copyBuffer"][:3]
    cw = [v["WRITE_SIZE"] for k, v, _ in write if k == "__amd_rocclr_copyBuffer"][:3]
    f_scale = copy / 1024 / statistics.median(cf)   # counter unit is KiB
    w_scale = copy / 1024 / statistics.median(cw)
    merged = [(k, {"bytes": f["FETCH_SIZE"] * f_scale * 1024 + w["WRITE_SIZE"] * w_scale * 1024}, r)
              for (k, f, r), (_, w, _) in zip(fetch, write)]
    lines = ["# Commands: rocprofv3 --pmc FETCH_SIZE -d F -o run --output-format csv -- python3 bench.py "
             "--pmc-workload --pmc-keys K; the same with WRITE_SIZE into W; then python bench.py --traffic-from "
             "F/run_counter_collection.csv W/run_counter_collection.csv K",
             f"# HBM bytes per launch = FETCH_SIZE*{f_scale:.4f} + WRITE_SIZE*{w_scale:.4f} (KiB -> bytes)",
             f"# scale factors: 64 MiB copy read FETCH_SIZE {statistics.median(cf):.1f} KiB, "
             f"WRITE_SIZE {statistics.median(cw):.1f} KiB"]
    for key, vals in _group(json.loads(Path(keys_json).read_text()), merged).items():
        lines.append(f"{key}={int(statistics.median(v[1]['bytes'] for v in vals))}  # {vals[0][0].split('(')[0]}")
    return "\n".join(lines) + "\n"


def mfma_from_pmc(pmc_csv: str, keys_json: str, command: str) -> str:
    """Markdown summary of the MFMA / LDS / clock counters of a
    ``--pmc-workload`` run: per kernel, the MFMA-busy fraction of all SIMD
    cycles (SQ_VALU_MFMA_BUSY_CYCLES over GRBM_GUI_ACTIVE per XCC times the
    SIMD count), the mean engine clock (GRBM_GUI_ACTIVE per XCC over the
    dispatch's duration), MFMA ops counted by the hardware against the
    algorithmic count, and LDS bank-conflict cycles over LDS-active
    cycles."""
    import statistics
    disp = _per_dispatch(pmc_csv)
    xcc, simds = 8, 256 * 4
    algo = {"gemm_i8_4096": 2.0 * 4096 ** 3, "ffn_gate_up": 2 * 2.0 * 2048 * 4096 * 11008,
            "ffn_down": 2.0 * 2048 * 4096 * 11008}
    lines = ["# MFMA utilisation, clock and LDS conflicts per kernel (rocprofv3 --pmc)", "",
             f"Command: `{command}`", "",
             "Per kernel, the median over its launches. MFMA busy = SQ_VALU_MFMA_BUSY_CYCLES / "
             "(GRBM_GUI_ACTIVE / 8 XCDs x 1024 SIMDs); clock = GRBM_GUI_ACTIVE / 8 / duration; "
             "MOPS x 512 = the operations the MFMA units counted (I8 or F16 MOPS); LDS conflict = "
             "SQ_LDS_BANK_CONFLICT / SQ_LDS_IDX_ACTIVE; waiting = SQ_WAIT_INST_ANY / SQ_WAVE_CYCLES (the "
             "share of wave-cycles a wave waited for any dependency: memory, LDS, MFMA results, barriers).",
             "",
             "| kernel (workload:config) | duration us | clock GHz | MFMA busy | counted ops / algorithmic | "
             "LDS conflict | waiting |", "|---|---:|---:|---:|---:|---:|---:|"]
    for key, vals in _group(json.loads(Path(keys_json).read_text()), disp).items():
        if not (key.startswith("gemm_i8_4096") or key.startswith("ffn_gate") or key.startswith("ffn_down")):
            continue
        rec = []
        for name, c, row in vals:
            d_ns = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
            gui = c.get("GRBM_GUI_ACTIVE", 0.0) / xcc
            busy = c.get("SQ_VALU_MFMA_BUSY_CYCLES", 0.0) / (gui * simds) if gui else float("nan")
            ops = 512.0 * (c.get("SQ_INSTS_VALU_MFMA_MOPS_I8", 0.0) + c.get("SQ_INSTS_VALU_MFMA_MOPS_F16", 0.0))
            lds = (c.get("SQ_LDS_BANK_CONFLICT", 0.0) / c["SQ_LDS_IDX_ACTIVE"]
                   if c.get("SQ_LDS_IDX_ACTIVE") else float("nan"))
            wait = (c.get("SQ_WAIT_INST_ANY", float("nan")) / c["SQ_WAVE_CYCLES"]
                    if c.get("SQ_WAVE_CYCLES") else float("nan"))
            rec.append((d_ns / 1e3 if d_ns else float("nan"), gui / d_ns if d_ns else float("nan"), busy, ops, lds,
                        wait))
        med = [statistics.median(r[i] for r in rec) for i in range(6)]
        base = next((v for k, v in algo.items() if key.startswith(k)), None)
        ratio = f"{med[3] / base:.3f}" if base else "-"
        lines.append(f"| {key} | {med[0]:.1f} | {med[1]:.3f} | {100 * med[2]:.1f}% | {ratio} | {100 * med[4]:.2f}% | "
                     f"{100 * med[5]:.1f}% |")
    return "\n".join(lines) + "\n"


def gemv_from_pmc(pmc_csv: str, keys_json: str, command: str) -> str:
    """Markdown summary of the decode-GEMV counters of a ``--pmc-workload``
    run (every GEMV config at M = 1, 4, 16, N = 11008, K = 4096): per config,
    the median over its launches of the duration, the launch shape (waves,
    VGPRs, LDS from the dispatch record), the share of wave-cycles spent
    waiting, vector-memory read instructions and L1-to-L2 read requests per
    launch against the weight's 1 KiB chunks, the L1's pending-stall cycles
    per wave and the texture-addresser busy share."""
    import statistics
    disp = _per_dispatch(pmc_csv)
    xcc = 8
    chunks = 11008 * 4096 // 1024
    lines = ["# Decode GEMV counters per config (rocprofv3 --pmc)", "",
             f"Command: `{command}`", "",
             "W8A16 GEMV, N = 11008, K = 4096, registered (fragment-packed) weight: 44,032 weight chunks of "
             "1 KiB, one 16-byte load per lane each. Per config and M, the median over its launches. "
             "waves = SQ_WAVES; VGPR / AGPR / LDS from the dispatch record (its VGPR field reads half the "
             "compiler's count for these kernels, rounded up to 4: 44 for the 82 VGPRs of packed_ct3_kw8, "
             "60 for the 114 of packed_ct3_kw16_e); waiting = SQ_WAIT_INST_ANY / "
             "SQ_WAVE_CYCLES; vmem reads = SQ_INSTS_VMEM_RD (wave instructions, weight and activation); "
             "L2 requests = TCP_TCC_READ_REQ_sum (64-byte requests from the L1s); pending stall = "
             "TCP_PENDING_STALL_CYCLES_sum per wave; TA busy = TA_BUSY_avr / (GRBM_GUI_ACTIVE / 8).", "",
             "| M | config | duration us | waves | VGPR | AGPR | LDS B | waiting | vmem reads / chunk | "
             "L2 requests / chunk | pending stall / wave | TA busy |",
             "|---:|---|---:|---:|---:|---:|---:|---:|---:|---:|---:|---:|"]
    for key, vals in _group(json.loads(Path(keys_json).read_text()), disp).items():
        if not key.startswith("gemv_w8a16_m"):
            continue
        m = key.split("_m", 1)[1].split(":", 1)[0]
        cfg = key.split(":", 1)[1].replace("gemv_", "")
        rec = []
        for name, c, row in vals:
            d_ns = int(row["End_Timestamp"]) - int(row["Start_Timestamp"])
            waves = c.get("SQ_WAVES", float("nan"))
            gui = c.get("GRBM_GUI_ACTIVE", 0.0) / xcc
            rec.append((d_ns / 1e3 if d_ns else float("nan"), waves,
                        c["SQ_WAIT_INST_ANY"] / c["SQ_WAVE_CYCLES"] if c.get("SQ_WAVE_CYCLES") else float("nan"),
                        c.get("SQ_INSTS_VMEM_RD", float("nan")) / chunks,
                        c.get("TCP_TCC_READ_REQ_sum", float("nan")) / chunks,
                        c.get("TCP_PENDING_STALL_CYCLES_sum", float("nan")) / waves if waves else float("nan"),
                        c.get("TA_BUSY_avr", float("nan")) / gui if gui else float("nan")))
        med = [statistics.median(r[i] for r in rec) for i in range(7)]
        row = vals[0][2]
        lines.append(f"| {m} | {cfg} | {med[0]:.2f} | {med[1]:.0f} | {row['VGPR_Count']} | {row['Accum_VGPR_Count']} | "
                     f"{row['LDS_Block_Size']} | {100 * med[2]:.1f}% | {med[3]:.2f} | {med[4]:.1f} | {med[5]:.0f} | "
                     f"{100 * med[6]:.1f}% |")
    return "\n".join(lines) + "\n"


def stats_from_trace(stats_csv: str, trace_csv: str, bench_json: str, command: str) -> str:
    """Markdown summary of a ``rocprofv3 --kernel-trace --stats`` run of
    the bench: the hx kernels of the stats CSV, the phases of the trace
    (consecutive dispatches of one kernel with one grid, >= 20 of them) and,
    beside the bench line's own live timing, the trace's mean for the
    headline kernel over its last phase of at least ``steps`` dispatches."""
    import csv
    import statistics
    rows = [r for r in csv.DictReader(open(stats_csv)) if "hx::" in r.get("Name", "")]
    lines = ["# Kernel durations, default `bench.py` run (rocprofv3 kernel trace)", "",
             f"Command: `{command}`", "",
             "The run includes the tile search (every compiled config of each tuned family is "
             "timed, so each config appears) and then the timed steps with the champion config.", "",
             "## Kernel statistics (hx kernels; durations in us)", "",
             "| kernel | calls | avg | min | max | % of GPU time |", "|---|---:|---:|---:|---:|---:|"]
    rows.sort(key=lambda r: -float(r["Percentage"]))
    for r in rows[:60]:
        lines.append(f"| `{r['Name']}` | {r['Calls']} | {float(r['AverageNs']) / 1e3:.2f} | "
                     f"{float(r['MinNs']) / 1e3:.2f} | {float(r['MaxNs']) / 1e3:.2f} | {float(r['Percentage']):.2f} |")
    trace = list(csv.DictReader(open(trace_csv)))
    trace.sort(key=lambda r: int(r["Start_Timestamp"]))
    phases = []
    for r in trace:
        name = r["Kernel_Name"]
        if "hx::" not in name:
            continue
        grid = r.get("Grid_Size") or ""
        if not grid and r.get("Grid_Size_X"):
            grid = str(int(r["Grid_Size_X"]) * int(r.get("Grid_Size_Y") or 1) * int(r.get("Grid_Size_Z") or 1))
        key = (name, grid)
        d = (int(r["End_Timestamp"]) - int(r["Start_Timestamp"])) / 1e3
        if phases and phases[-1][0] == key:
            phases[-1][1].append(d)
        else:
            phases.append((key, [d]))
    lines += ["", "## Phases of the trace (>= 20 consecutive dispatches; us)", "",
              "| kernel | grid (work-items) | dispatches | mean | median |", "|---|---:|---:|---:|---:|"]
    for (name, grid), ds in phases:
        if len(ds) >= 20:
            lines.append(f"| `{name.replace('void ', '')}` | {grid} | {len(ds)} | {statistics.mean(ds):.2f} | "
                         f"{statistics.median(ds):.2f} |")
    line = json.loads(Path(bench_json).read_text().strip().splitlines()[-1])
    head = line["config"]["kernel"]
    steps = int(line["steps"])
    # the headline config's kernel with no edge tiles and a [N][K] B
    import re
    m = re.match(r"(\d+)x(\d+)_w(\d+)x(\d+)", head)
    prefix = f"hx::gemm_kernel<0, {m[1]}, {m[2]}, {m[3]}, {m[4]}, 0, " if m else "hx::gemm_kernel<0, "
    warm = int(line.get("warmup", 0))
    cand = [(k, ds) for k, ds in phases
            if k[0].replace("void ", "").startswith(prefix) and ", false, false," in k[0] and len(ds) >= steps]
    # the headline's own phase: its warmup and timed steps between the two
    # marker launches (exactly warmup + steps dispatches); else the last
    # long enough phase of that kernel
    exact = [(k, ds) for k, ds in cand if len(ds) == warm + steps]
    lines += ["", "## Agreement with the bench line", "",
              f"The bench line (same process, under the profiler) reports {line['kernel_us']} us per launch for "
              f"the headline kernel ({head}), from one HIP event pair around its {steps} timed steps on the "
              f"launch stream."]
    if exact:
        (name, grid), ds = exact[0]
        timed = ds[-steps:]
        lines.append(f"The trace's phase of that kernel with the bench's {warm} warmup and {steps} timed dispatches "
                     f"(`{name.replace('void ', '')}`): the timed {steps} have mean {statistics.mean(timed):.2f} us, "
                     f"median {statistics.median(timed):.2f} us.")
    elif cand:
        (name, grid), ds = cand[-1]
        lines.append(f"The trace's last phase of that kernel with >= {steps} dispatches ({len(ds)} dispatches, "
                     f"`{name.replace('void ', '')}`) has mean {statistics.mean(ds):.2f} us, median "
                     f"{statistics.median(ds):.2f} us.")
    return "\n".join(lines) + "\n"


def ceilings(hx=None) -> dict:
    """What this box sustains, timed with HIP events over back-to-back
    launches (the way every kernel of the bench line is timed) using the
    probes of libhxprobe.so: the launch period of an empty kernel, a
    streaming read and a copy (rotating over copies larger than the 256 MB
    MALL, best of a sweep of grid sizes), and int8 MFMA issue on register
    operands with LDS reads (6 per 8 MFMAs is the GEMM's 128x64 wave tile)
    and L2-resident global loads beside it."""
    import torch
    import importlib.util
    spec = importlib.util.spec_from_file_location("_hx_build", ROOT / "hexagon-mlir_amd" / "build.py")
    b = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(b)
    lib = ctypes.CDLL(str(b.build_probe()))
    vp, i64, ci = ctypes.c_void_p, ctypes.c_int64, ctypes.c_int
    lib.hxp_empty.argtypes = [vp]
    lib.hxp_read.argtypes = [vp, i64, ci, vp, vp]
    lib.hxp_copy.argtypes = [vp, vp, i64, ci, vp]
    lib.hxp_mfma_i8.argtypes = [ci, ci, ci, ci, vp, vp, ctypes.POINTER(ctypes.c_double), vp]
    dev = torch.device("cuda:0")
    stream = lambda: ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)  # noqa: E731
    out = {}
    sink = torch.zeros(1 << 16, dtype=torch.int32, device=dev)
    gr = torch.Generator(device=dev).manual_seed(7)
    ms, _ = event_timed([lambda: lib.hxp_empty(stream())], 2000)
    out["empty_launch_period_us"] = round(ms * 1e3, 3)

    def sweep(label, nbytes, fn_of):
        best = None
        for blocks in (512, 1024, 2048, 4096, 8192):
            calls = fn_of(blocks)
            ms, _ = event_timed(calls, 200)
            if best is None or ms < best[0]:
                best = (ms, blocks)
        ms, blocks = best
        out[label] = {"bytes": nbytes, "us_per_launch": round(ms * 1e3, 3),
                      "GB_s": round(nbytes / (ms * 1e-3) / 1e9, 1), "blocks": blocks}

    for mb in (45, 64, 256):
        nbytes = (45_140_992 if mb == 45 else mb << 20)
        copies = max(1, min(16, -(-(600 << 20) // nbytes)))
        # random words: the HBM stream rate does not depend on the data (a
        # 45 MB read of ones, zeros or random words: 7.74-7.78 us)
        bufs = [torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev, generator=gr)
                for _ in range(copies)]
        sweep(f"read_{mb}MB", nbytes, lambda blocks, bufs=bufs, nbytes=nbytes: [
            (lambda b=b: lib.hxp_read(ctypes.c_void_p(b.data_ptr()), nbytes, blocks,
                                      ctypes.c_void_p(sink.data_ptr()), stream())) for b in bufs])
        del bufs
    # the decode GEMV's weight read in the GEMV's own launch shape (no
    # arithmetic), 12 rotating copies like the GEMV's bench line
    lib.hxp_read_gemv_shape.argtypes = [vp, i64, vp, ci, vp, vp]
    gbytes = 11008 * 4096
    wcopies = [torch.randint(-2**31, 2**31 - 1, (gbytes // 4,), dtype=torch.int32, device=dev, generator=gr)
               for _ in range(12)]
    scales = torch.ones(11008, dtype=torch.float32, device=dev)
    ms, _ = event_timed([(lambda w=w: lib.hxp_read_gemv_shape(ctypes.c_void_p(w.data_ptr()), gbytes,
                                                              ctypes.c_void_p(scales.data_ptr()), 11008,
                                                              ctypes.c_void_p(sink.data_ptr()), stream()))
                         for w in wcopies], 400)
    out["read_45MB_gemv_shape"] = {"bytes": gbytes, "us_per_launch": round(ms * 1e3, 3),
                                   "GB_s": round(gbytes / (ms * 1e-3) / 1e9, 1), "blocks": -(-gbytes // (3 * 65536))}
    # the same read in the launch shapes of other GEMV configs (tiles per
    # workgroup, waves)
    lib.hxp_read_tiles.argtypes = [ci, ci, vp, i64, vp, ci, vp, vp]
    for ct, kw in ((3, 8), (1, 8), (1, 4)):
        ms, _ = event_timed([(lambda w=w, ct=ct, kw=kw: lib.hxp_read_tiles(
            ct, kw, ctypes.c_void_p(w.data_ptr()), gbytes, ctypes.c_void_p(scales.data_ptr()), 11008,
            ctypes.c_void_p(sink.data_ptr()), stream())) for w in wcopies], 400)
        out[f"read_45MB_gemv_shape_ct{ct}_kw{kw}"] = {
            "bytes": gbytes, "us_per_launch": round(ms * 1e3, 3), "GB_s": round(gbytes / (ms * 1e-3) / 1e9, 1),
            "blocks": -(-gbytes // (ct * 65536))}
    del wcopies
    nbytes = 64 << 20
    pairs = [(torch.randint(-2**31, 2**31 - 1, (nbytes // 4,), dtype=torch.int32, device=dev, generator=gr),
              torch.empty(nbytes // 4, dtype=torch.int32, device=dev))
             for _ in range(6)]
    sweep("copy_64MiB_in_64MiB_out", 2 * nbytes, lambda blocks: [
        (lambda s_=s_, d_=d_: lib.hxp_copy(ctypes.c_void_p(s_.data_ptr()), ctypes.c_void_p(d_.data_ptr()), nbytes,
                                           blocks, stream())) for s_, d_ in pairs])
    # the same bytes in the row kernels' pattern: one workgroup per 8 KiB row
    lib.hxp_copy_rows.argtypes = [vp, vp, i64, vp]
    ms, _ = event_timed([(lambda s_=s_, d_=d_: lib.hxp_copy_rows(
        ctypes.c_void_p(s_.data_ptr()), ctypes.c_void_p(d_.data_ptr()), nbytes, stream())) for s_, d_ in pairs], 200)
    out["copy_64MiB_row_pattern"] = {"bytes": 2 * nbytes, "us_per_launch": round(ms * 1e3, 3),
                                     "GB_s": round(2 * nbytes / (ms * 1e-3) / 1e9, 1), "blocks": nbytes // 8192}
    del pairs
    ops = ctypes.c_double()
    gbuf = torch.ones(1 << 18, dtype=torch.int32, device=dev)  # 1 MiB, L2-resident
    for nr, ng in ((0, 0), (2, 0), (4, 0), (6, 0), (0, 2), (0, 4), (0, 6), (4, 2), (2, 4)):
        call = lambda nr=nr, ng=ng: lib.hxp_mfma_i8(  # noqa: E731
            256, 4000, nr, ng, ctypes.c_void_p(gbuf.data_ptr()), ctypes.c_void_p(sink.data_ptr()),
            ctypes.byref(ops), stream())
        ms, _ = event_timed([call], 20)
        out[f"mfma_i8_{nr}_lds_{ng}_vmem_per_8"] = {
            "us_per_launch": round(ms * 1e3, 2), "TOPS": round(ops.value / (ms * 1e-3) / 1e12, 1),
            "frac_of_5000": round(ops.value / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}
    lib.hxp_mfma4_i8.argtypes = [ci, ci, ci, vp, ctypes.POINTER(ctypes.c_double), vp]
    for nr in (0, 4, 8):
        call = lambda nr=nr: lib.hxp_mfma4_i8(256, 4000, nr, ctypes.c_void_p(sink.data_ptr()),  # noqa: E731
                                              ctypes.byref(ops), stream())
        ms, _ = event_timed([call], 20)
        out[f"mfma_i8_4waves_{nr}_lds_per_16"] = {
            "us_per_launch": round(ms * 1e3, 2), "TOPS": round(ops.value / (ms * 1e-3) / 1e12, 1),
            "frac_of_5000": round(ops.value / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}
    # the GEMM's interleaved schedule against ping-pong (two groups of four
    # waves alternating MFMA and read bursts between workgroup barriers)
    lib.hxp_mfma_sched_i8.argtypes = [ci, ci, ci, vp, ctypes.POINTER(ctypes.c_double), vp]
    sched = {0: ("interleaved", 1, 4096), 1: ("interleaved", 2, 2048), 2: ("pingpong", 1, 4096),
             3: ("pingpong_setprio", 1, 4096), 4: ("pingpong", 2, 2048), 5: ("pingpong_setprio", 2, 2048),
             6: ("pingpong_setprio", 4, 1024)}
    for kind, (name, rounds, phases) in sched.items():
        call = lambda kind=kind, phases=phases: lib.hxp_mfma_sched_i8(  # noqa: E731
            kind, 256, phases, ctypes.c_void_p(sink.data_ptr()), ctypes.byref(ops), stream())
        ms, _ = event_timed([call], 20)
        out[f"mfma_i8_6_lds_per_8_{name}_{8 * rounds}_mfma_per_phase"] = {
            "us_per_launch": round(ms * 1e3, 2), "TOPS": round(ops.value / (ms * 1e-3) / 1e12, 1),
            "frac_of_5000": round(ops.value / (ms * 1e-3) / 1e12 / PEAK_INT8_TOPS, 4)}
    if hx is not None:
        out.update(operand_data_ceiling(hx))
    return out


def operand_data_ceiling(hx) -> dict:
    """The headline product (hx_gemm_i8, 4096^3, fp16 dequant, the same
    config and binary as the bench line) timed on operands of different
    value ranges.  The arithmetic and every memory access are identical;
    only the bits the MFMA arrays switch differ, so the spread is the chip's
    power and current management reacting to the data."""
    import torch
    M = N = K = 4096
    dev = torch.device("cuda:0")
    g = torch.Generator(device=dev).manual_seed(99)
    sa = torch.empty(M, dtype=torch.float32, device=dev).uniform_(0.001, 0.02, generator=g)
    sb = torch.empty(N, dtype=torch.float32, device=dev).uniform_(0.001, 0.02, generator=g)
    c = torch.empty((M, N), dtype=torch.float16, device=dev)
    cfg_idx = hx.config_lookup(1, M, N, K)
    res = {}
    for label, lo, hi in (("zero", 0, 0), ("one", 1, 1), ("uniform_-1_1", -1, 1), ("uniform_-15_15", -15, 15),
                          ("uniform_-127_127", -127, 127)):
        a = torch.randint(lo, hi + 1, (M, K), dtype=torch.int8, device=dev, generator=g)
        bt = torch.randint(lo, hi + 1, (N, K), dtype=torch.int8, device=dev, generator=g)
        step = hx.bind_gemm_i8(a, bt, c, b_layout="nk", row_scale=sa, col_scale=sb)
        ms, _ = event_timed([step], 200)
        tops = 2.0 * M * N * K / (ms * 1e-3) / 1e12
        res[f"gemm_i8_4096_dequant_operands_{label}"] = {
            "us_per_launch": round(ms * 1e3, 2), "TOPS": round(tops, 1),
            "frac_of_5000": round(tops / PEAK_INT8_TOPS, 4),
            "config": hx.config_get(1, cfg_idx)["name"] if cfg_idx >= 0 else "default"}
        del a, bt
    # the W8A16 product of the FFN's gate projection (f16 MFMA on int8 weights
    # widened in registers): activations and weights zero, or as configs[4]
    Mw, Nw, Kw = 2048, 11008, 4096
    s16 = torch.empty(Nw, dtype=torch.float16, device=dev).uniform_(0.001, 0.02, generator=g)
    y = torch.empty((Mw, Nw), dtype=torch.float16, device=dev)
    for label, zero in (("zero", True), ("ffn_data", False)):
        x = torch.zeros((Mw, Kw), dtype=torch.float16, device=dev) if zero else \
            torch.randn((Mw, Kw), dtype=torch.float16, device=dev, generator=g)
        w = torch.zeros((Kw, Nw), dtype=torch.int8, device=dev) if zero else \
            torch.randint(-127, 128, (Kw, Nw), dtype=torch.int8, device=dev, generator=g)
        rw = hx.ResidentWeight(w, s16, layout="kn")
        ms, _ = event_timed([hx.bind_matmul_resident(x, rw, y)], 50)
        tf = 2.0 * Mw * Nw * Kw / (ms * 1e-3) / 1e12
        res[f"gemm_w8a16_2048x11008x4096_operands_{label}"] = {
            "us_per_launch": round(ms * 1e3, 2), "TFLOPS": round(tf, 1),
            "frac_of_2500": round(tf / PEAK_F16_TFLOPS, 4)}
        rw.release()
        del x, w
    # the whole SwiGLU FFN block with zero operands and with the
    # bench line's data (the same untuned configurations in both)
    T, H, I = 2048, 4096, 11008
    for label, zero in (("zero", True), ("ffn_data", False)):
        def wt(k, n):
            w = torch.zeros((k, n), dtype=torch.int8, device=dev) if zero else \
                torch.randint(-127, 128, (k, n), dtype=torch.int8, device=dev, generator=g)
            s = torch.empty(n, dtype=torch.float16, device=dev).uniform_(0.5, 1.5, generator=g) / (127 * (k / 3) ** 0.5)
            return hx.ResidentWeight(w, s.half(), layout="kn")
        ws = [wt(H, I), wt(H, I), wt(I, H)]
        x = torch.zeros((T, H), dtype=torch.float16, device=dev) if zero else \
            torch.randn((T, H), dtype=torch.float16, device=dev, generator=g)
        gamma = torch.randn(H, dtype=torch.float16, device=dev, generator=g) * 0.1 + 1.0
        y = torch.empty_like(x)
        ms, _ = event_timed([lambda: hx.swiglu_ffn(x, gamma, 1e-6, *ws, out=y)], 20)
        tf = 3 * 2.0 * T * H * I / (ms * 1e-3) / 1e12
        res[f"swiglu_ffn_2048x4096x11008_operands_{label}"] = {
            "us_per_launch": round(ms * 1e3, 1), "TFLOPS": round(tf, 1),
            "frac_of_2500": round(tf / PEAK_F16_TFLOPS, 4)}
        for w in ws:
            w.release()
        del x, y
    return res


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--only", choices=["headline", "all"], default="all")
    ap.add_argument("--no-tune", action="store_true",
                    help="time the untuned default configs (skip the tile search)")
    ap.add_argument("--pmc-workload", action="store_true",
                    help="launch each benchmarked kernel a few times for rocprofv3 --pmc")
    ap.add_argument("--ffn-decode", action="store_true",
                    help="the SwiGLU FFN block at decode token counts, markdown on stdout, exit")
    ap.add_argument("--gemv-ab", action="store_true",
                    help="interleaved A/B of the decode GEMV default candidates, markdown on stdout, exit")
    ap.add_argument("--vendor", action="store_true",
                    help="only the vendor GEMMs beside hx at 4096^3 (for a kernel trace), JSON on stdout, exit")
    ap.add_argument("--rows-ab", action="store_true",
                    help="interleaved A/B of the row configurations, markdown on stdout, exit")
    ap.add_argument("--ceilings", action="store_true",
                    help="time the libhxprobe probes (launch gap, read, copy, MFMA issue), print JSON, exit")
    ap.add_argument("--pmc-keys", metavar="JSON",
                    help="with --pmc-workload: write the launch sequence the counter parsers read")
    ap.add_argument("--traffic-from", nargs=3, metavar=("FETCH_CSV", "WRITE_CSV", "KEYS_JSON"),
                    help="print the traffic.txt lines of two --pmc-workload counter CSVs and exit")
    ap.add_argument("--stats-from", nargs=4, metavar=("STATS_CSV", "TRACE_CSV", "BENCH_JSON", "COMMAND"),
                    help="markdown summary of a rocprofv3 --kernel-trace --stats run of the bench")
    ap.add_argument("--gemv-from", nargs=3, metavar=("PMC_CSV", "KEYS_JSON", "COMMAND"),
                    help="print the decode-GEMV counter summary of a --pmc-workload counter CSV and exit")
    ap.add_argument("--mfma-from", nargs=3, metavar=("PMC_CSV", "KEYS_JSON", "COMMAND"),
                    help="print the MFMA counter summary of a --pmc-workload counter CSV (and the "
                         "command that made it) and exit")
    args = ap.parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build runs on one GPU; --gpus {args.gpus} is not supported "
              "(multi-GPU sharding is designed, not built: one GPU's shard is what this bench measures)", file=sys.stderr)
        return 2

    if args.traffic_from:
        print(traffic_from_pmc(*args.traffic_from), end="")
        return 0
    if args.stats_from:
        print(stats_from_trace(*args.stats_from), end="")
        return 0
    if args.mfma_from:
        print(mfma_from_pmc(*args.mfma_from), end="")
        return 0
    if args.gemv_from:
        print(gemv_from_pmc(*args.gemv_from), end="")
        return 0
    import torch
    from __graft_entry__ import load_package
    hx = load_package()
    if not torch.cuda.is_available():
        print("bench.py: no GPU visible", file=sys.stderr)
        return 1
    rc = hx.load().hx_init()
    if rc != 0:
        print(f"bench.py: hx_init failed: {hx._abi.last_error()}", file=sys.stderr)
        return 1
    if args.ceilings:
        print(json.dumps(ceilings(hx)), flush=True)
        return 0
    if args.gemv_ab:
        print(gemv_ab(hx), end="", flush=True)
        return 0
    if args.ffn_decode:
        print(ffn_decode_table(hx), end="", flush=True)
        return 0
    if args.rows_ab:
        print(rows_ab(hx), end="", flush=True)
        return 0
    if args.vendor:
        M = N = K = 4096
        dev = torch.device("cuda:0")
        g = torch.Generator(device=dev).manual_seed(1234)
        a = torch.randint(-127, 128, (M, K), dtype=torch.int8, device=dev, generator=g)
        bt = torch.randint(-127, 128, (N, K), dtype=torch.int8, device=dev, generator=g)
        print(json.dumps(bench_vendor_gemms(hx, (a, bt, None, None))), flush=True)
        return 0
    if args.pmc_workload:
        pmc_workload(hx, args.pmc_keys)
        return 0

    log("[bench] int8 GEMM 4096^3 + dequant")
    tune_on = not args.no_tune
    h = bench_gemm_i8(hx, args.steps, args.warmup, tune_on=tune_on)
    log(f"[bench] int8 GEMM: {h['tops']:.1f} TOPS wall, {h['tops_kernel']:.1f} TOPS kernel, "
        f"{h['kernel_ms']*1e3:.1f} us/launch, parity={h['parity_sampled_rows_bitexact']}")
    secondary = []
    if args.only == "all":
        log("[bench] int8 GEMM 4096^3, int32 out")
        secondary.append(bench_gemm_i8_i32(hx, h["inputs"]))
        log("[bench] int8 GEMM 4096^3, [K][N] B in place")
        secondary.append(bench_gemm_i8_kn(hx, h["inputs"]))
        log("[bench] vendor GEMMs beside hx")
        secondary.append(bench_vendor_gemms(hx, h["inputs"]))
        log("[bench] W8A16 GEMV")
        secondary += bench_gemv(hx, tune_on=tune_on)
        log("[bench] W8A16 GEMV, down-projection shape")
        secondary += bench_gemv_down(hx)
        log("[bench] row ops")
        secondary += bench_rows(hx)
        secondary.append(bench_rows_long(hx))
        log("[bench] fp16 GEMM 256^3")
        secondary.append(bench_gemm_f16_small(hx))
        log("[bench] fp16 matmul at the reference's published shapes")
        secondary += bench_reference_shapes(hx)
        log("[bench] fp16 decode at the reference tuner's decode shapes")
        secondary += bench_f16_decode(hx)
        log("[bench] SwiGLU FFN")
        secondary.append(bench_ffn(hx, tune_on=tune_on))
        log("[bench] attention")
        secondary += bench_attention(hx)
        for s in secondary:
            log(f"[bench]   {s['workload']}: {s['value']} {s['unit']}")
    cpu = None
    if not args.no_cpu:
        import oracle
        march = oracle.use_native_build()
        log(f"[bench] CPU baseline (oracle port, -march=native = {march})")
        cpu = cpu_baseline_gemm_i8(h["inputs"], march, gpu_out=h["output"])
        log(f"[bench] CPU: {cpu['value']} TOPS on {cpu['cores']} threads")
        if secondary:
            sec_cpu = cpu_baselines_secondary(march)
            keys = {"W8A16 GEMV M=1 ": "gemv_m1", "W8A16 GEMV M=4 ": "gemv_m4",
                    "W8A16 GEMV M=16 N=11008 ": "gemv_m16", "W8A16 GEMV M=16 N=4096 ": "gemv_down",
                    "softmax fp16 [8192": "softmax", "softmax fp16 [2048 x 128256]": "softmax_vocab",
                    "rmsnorm fp16": "rmsnorm", "fp16 GEMM 256^3": "gemm_f16_256",
                    "SwiGLU FFN": "ffn"}
            keys.update({f"fp16 matmul {M}x{N}x{K} ": f"ref_{M}x{N}x{K}" for (M, N, K) in REF_SHAPES})
            keys.update({f"fp16 decode {M}x{N}x{K},": f"dec_{M}x{N}x{K}" for (M, N, K) in ((1, 8192, 8192),
                                                                                       (1, 4096, 16384))})
            keys.update({"attention Z=1 H=1 N=1024 D=64 fp16": "attn_ref",
                         "attention Z=4 H=16 N=2048 D=128 fp16": "attn_mh",
                         "attention Z=4 H=16 N=2048 D=128 causal fp16": "attn_mh_causal"})
            for sec in secondary:
                for prefix, key in keys.items():
                    if sec["workload"].startswith(prefix):
                        sec["cpu_baseline"] = sec_cpu[key]
                if sec["workload"].startswith("int8 GEMM M=N=K="):
                    # the same product as the headline: its CPU sample
                    sec["cpu_baseline"] = dict(cpu, note="the headline's CPU sample (same product)")
            log("[bench] CPU secondary baselines done")

    line = {
        "metric": METRIC,
        "value": round(h["tops"], 2),
        "unit": "TOPS",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "int8",
        "data": "synthetic (seeded uniform int8 operands and fp32 scales generated on the device)",
        "config": {"workload": "int8 GEMM M=N=K=4096, int32 accumulate, per-row/per-col fp32 "
                               "scales -> fp16 (BASELINE configs[1])",
                   "M": 4096, "N": 4096, "K": 4096, "b_layout": "nk (resident weight image)",
                   "kernel": h["kernel"], "parallelism": "single GPU"},
        "roofline": roofline("mfma", h["tops_kernel"], PEAK_INT8_TOPS, "TFLOP/s",
                             traffic_of(f"gemm_i8_4096_dequant_f16:{h['kernel']}")),
        "roofline_note": "int8 ops counted as 2 per MAC; achieved = 2*4096^3 / mean device time "
                         "per launch, one HIP event pair around the K back-to-back steps on the "
                         "launch stream",
        "kernel_us": round(h["kernel_ms"] * 1e3, 3),
        "spread": dict(h["spread"].spread(), note="7 more timed regions of the same launches after the "
                                                  "timed steps; the figure is the steps' own region"),
        "clock": h["clock"],
        "zero_operands": h["zero_operands"],
        "queue_fed": h["queue_fed"],
        "parity": {"int8_sampled_rows_bitexact": h["parity_sampled_rows_bitexact"],
                   "all_elements_bitexact": (cpu or {}).get("gpu_output_bitexact_all_elements")},
        "tune": h["tune"],
        "plan": h["plan"],
        "cpu_baseline": cpu,
        "secondary": secondary,
    }
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
