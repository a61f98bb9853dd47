#!/usr/bin/env python3
"""Throughput of the fused forward+adjoint Monte-Carlo replay on one MI355X.

Workload: arithmetic-average Asian call under GBM, 252 daily fixings, ATM 1y
(S0=K=100, sigma=0.20, r=0.03, T=1), value + 5 first-order Greeks, 2,000,000
scenarios per step, Philox seed 42; the headline is fp64 and the fp32 run is
reported beside it. The engine's default derivative mode (the lowering's cost
model: tangent for this tape) is the headline; the reverse-sweep kernel of the
same tape is timed beside it under "reverse". A step is one replay (one
dispatch through the C ABI: replay kernel, deterministic finishing kernel,
sums copied back) over a fresh range of 2,000,000 scenarios; inputs are
resident on the device before timing starts.

Prints one JSON line. `roofline` prices the replay kernel against the VALU
peak with the NT-FLOP v1 algorithmic count (nablatensor_amd/flops.py), using
the kernel's own HIP-event duration on its stream. `cpu_baseline` times the
CPU oracle (a C restatement of the reference's scalar `cpu` engine, OpenMP
over contiguous path ranges) on this host on a bounded sample; the
reference's Java engines cannot run here (no JDK). `workloads` reports the
other benchmark configurations (European, barrier, Heston-Asian, worst-of)
measured in the same run with fewer timed steps (--no-workloads skips them).
"""
from __future__ import annotations

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

WORKLOAD = "Asian call, GBM, 252 fixings, ATM 1y, value + 5 Greeks"
MODES = {1: "reverse", 2: "tangent"}
# The reference's rocm engine, fp64, same tape, 2,000,000 scenarios, seed 42, on a
# Radeon 780M (gfx1103): docs/examples/asian-greeks.md:43.
REFERENCE_ROCM_FP64 = 2.16e6


def workload_tape(name: str, coefficients: int = 24):
    from nablatensor_amd import workloads

    if name == "asian_weekdays":
        return workloads.schedule_tapes()[name].flat()
    if name == "local_vol":
        return workloads.local_vol_asian_tape(coefficients).flat()
    return workloads.workload_tapes()[name].flat()


# The committed counter summary of each workload's replay kernel (profiles/).
COUNTER_FILES = {"C1": "european1", "C2": "asian252", "C3": "barrier252", "C4": "heston_asian504",
                 "C5": "worstof16", "asian_weekdays": "asian_weekdays252", "local_vol": "local_vol24"}


def measured_counters(workload: str, precision: str, info: dict, grid: int | None = None) -> dict:
    """From the committed rocprofv3 summary of this workload and precision, the
    lines that match this kernel (derivative mode, checkpoint policy, segment
    length, straight-line segments and VGPRs, and, when `grid` is given, the
    blocks the dispatch launches): `traffic` (HBM bytes per dispatch,
    FETCH_SIZE and WRITE_SIZE copy-calibrated) and `executed` (executed FLOPs
    per scenario from the VALU counters)."""
    out = {}
    path = ROOT / "profiles" / f"nt_replay_{COUNTER_FILES.get(workload, workload)}_{precision}_counters.md"
    if not path.exists():
        return out
    want = {"mode": info["mode"], "checkpoint": info["checkpoint"], "seg_len": info["seg_len"],
            "segments": info["n_segments"], "vgprs": info["vgprs"]}
    if grid is not None:
        want["grid"] = grid
    for line in path.read_text().splitlines():
        kind = line.split(":", 1)[0]
        if kind not in ("traffic", "executed"):
            continue
        kv = dict(item.split("=") for item in line.split()[1:])
        if all(k in kv and int(kv[k]) == v for k, v in want.items()):
            out[kind] = {k: float(v) for k, v in kv.items() if k not in want}
            out[kind]["source"] = str(path.relative_to(ROOT))
    return out


def cost_model(source: str) -> dict | None:
    """The lowering's estimate of each derivative mode's work per path (VALU
    instructions; the `// nt-cost:` line of the generated source), which
    picks the mode when none is forced."""
    for line in source.splitlines():
        if line.startswith("// nt-cost:"):
            return {k: int(v) for k, v in (kv.split("=") for kv in line.split()[2:])}
    return None


def measure(rocm, flat, precision, paths, steps, warmup, seed, policy, seg, mode=0, ramp=0.5, workload="C2",
            waves=0, max_blocks=0, basis=0, roll=1, block=0):
    from nablatensor_amd import flops

    with rocm.Executable(flat, rocm.options(precision, checkpoint=policy, seg_len=seg, mode=mode, waves=waves,
                                                max_blocks=max_blocks, basis=basis, roll=roll, block=block)) as x:
        info = x.info()
        grid = x.grid(paths)[0]
        cost = cost_model(x.source())
        # The GPU's clocks ramp under sustained load: replay for `ramp` seconds
        # (untimed) before the warmup steps, so a short --warmup does not time
        # a cold device.
        t_ramp = time.perf_counter()
        while time.perf_counter() - t_ramp < ramp:
            x.replay(paths, 0, seed)
        for w in range(warmup):
            x.replay(paths, w * paths, seed)
        replay_ms, kernel_ms = [], []
        t0 = time.perf_counter()
        for k in range(steps):
            _, tm = x.replay(paths, (warmup + k) * paths, seed)
            replay_ms.append(tm["replay_ms"])
            kernel_ms.append(tm["kernel_ms"])
        wall = time.perf_counter() - t0
    fl = flops.flops_per_scenario(flat, precision)
    avg_replay_s = sum(replay_ms) / len(replay_ms) / 1e3
    # The committed counter summaries are per workload at the scenarios per dispatch it names.
    from nablatensor_amd import workloads

    counted = measured_counters(workload, precision, info, grid) if paths == workloads.DESCRIPTIONS[workload][1] else {}
    traffic = counted.get("traffic")
    executed = counted.get("executed")
    achieved = fl * paths / avg_replay_s / 1e12
    peak = flops.PEAK_TFLOPS[precision]
    ex_achieved = None if executed is None else executed["flops_per_scenario"] * paths / avg_replay_s / 1e12
    return {
        "value": paths * steps / wall,
        "ms_per_step": wall / steps * 1e3,
        "kernel_ms": sum(kernel_ms) / len(kernel_ms),
        "replay_kernel_ms": avg_replay_s * 1e3,
        "kernel_scenarios_per_s": paths / avg_replay_s,
        "roofline": {"bound": "valu", "kernel": "nt_replay", "achieved": achieved, "peak": peak,
                     "unit": "TFLOP/s", "frac": achieved / peak,
                     "traffic": None if traffic is None else traffic["bytes"],
                     "traffic_source": None if traffic is None else traffic["source"],
                     "executed_flops_per_scenario": None if executed is None else executed["flops_per_scenario"],
                     "executed_achieved": ex_achieved,
                     "executed_frac": None if ex_achieved is None else ex_achieved / peak,
                     "valu_issue": None if executed is None else executed.get("valu_issue"),
                     "executed_source": None if executed is None else executed["source"],
                     "algorithmic_bytes": 8 * (len(flat["input_node"]) + grid * (2 + len(flat["input_node"]))),
                     "flops_per_scenario": fl, "convention": "NT-FLOP v1"},
        "kernel": {**{k: info[k] for k in ("vgprs", "sgprs", "scratch_bytes", "lds_bytes", "loop_period",
                                           "loop_iters", "seg_len", "n_segments", "checkpoint", "tape_slots",
                                           "grid_cap")},
                   "grid": grid, "mode": MODES[info["mode"]], "cost_model": cost},
    }


def measure_markets(rocm, flat, precision, paths, steps, warmup, seed, markets, ramp=0.5, adjoints=True):
    """A revaluation ladder: `markets` input sets (the recorded inputs scaled by
    1 + 1% * (m - markets/2)) priced per dispatch from shared draws (with the
    Greeks, or prices only)."""
    import numpy as np

    x0 = np.array(flat["recorded_inputs"])
    sets = np.stack([x0 * (1.0 + 0.01 * (m - markets // 2)) for m in range(markets)])
    with rocm.Executable(flat, rocm.options(precision, adjoints=adjoints)) as x:
        info = x.info()
        t_ramp = time.perf_counter()
        while time.perf_counter() - t_ramp < ramp:
            x.replay_many(sets, paths, 0, seed)
        for w in range(warmup):
            x.replay_many(sets, paths, w * paths, seed)
        replay_ms = []
        t0 = time.perf_counter()
        for k in range(steps):
            _, tm = x.replay_many(sets, paths, (warmup + k) * paths, seed)
            replay_ms.append(tm["replay_ms"])
        wall = time.perf_counter() - t0
        single = x.replay(paths, 0, seed)[1]["replay_ms"]
    avg = sum(replay_ms) / len(replay_ms)
    return {"value": paths * markets * steps / wall, "ms_per_step": wall / steps * 1e3, "replay_kernel_ms": avg,
            "single_market_kernel_ms": single, "markets": markets, "mode": MODES[info["mode"]],
            "speedup_vs_separate": markets * single / avg}


def adjoint_vs_bump(rocm, flat, paths, seed, repeats=3, ramp=0.2) -> dict:
    """The adjoint against bump-and-revalue on the headline tape (fp64): one
    dispatch that returns the value and all 5 Greeks, against the 1 + 2 x 5
    price-only dispatches of a central bump with common random numbers,
    h_j = 5e-3 max(1, |x_j|) (BumpCrossCheck.java:33-49), and against the same
    11 input sets priced in one multi-market dispatch that shares the draws.
    Each is timed as the reference's Benchmarks.adjointVsBump does
    (Benchmarks.java:69-90): a warm run, then the best of 3, wall clock on the
    host per request, with the kernels' HIP-event time beside it."""
    import numpy as np

    from nablatensor_amd import bumps

    sets, h = bumps.central_bump_sets(flat["recorded_inputs"])

    def best(run):
        run()
        return min((run() for _ in range(repeats)), key=lambda r: r[0])

    with rocm.Executable(flat, rocm.options("fp64")) as ad, \
            rocm.Executable(flat, rocm.options("fp64", adjoints=False)) as po:
        t_ramp = time.perf_counter()
        while time.perf_counter() - t_ramp < ramp:
            ad.replay(paths, 0, seed)

        def adjoint():
            t0 = time.perf_counter()
            sums, tm = ad.replay(paths, 0, seed)
            return time.perf_counter() - t0, tm["kernel_ms"], sums[2:] / paths

        def separate():
            t0, kernel, prices = time.perf_counter(), 0.0, []
            for x in sets:
                po.set_inputs(x)
                sums, tm = po.replay(paths, 0, seed)
                kernel += tm["kernel_ms"]
                prices.append(sums[0] / paths)
            return time.perf_counter() - t0, kernel, np.array(prices)

        def shared():
            t0 = time.perf_counter()
            sums, tm = po.replay_many(sets, paths, 0, seed)
            return time.perf_counter() - t0, tm["kernel_ms"], sums[:, 0] / paths

        a, b, m = best(adjoint), best(separate), best(shared)
        po.set_inputs(sets[0])
        one = best(lambda: (lambda t0, r: (time.perf_counter() - t0, r[1]["kernel_ms"], None))(
            time.perf_counter(), po.replay(paths, 0, seed)))
    fd = bumps.bump_greeks(b[2], h)
    return {"scenarios": paths, "relative_bump": 5e-3, "replays": len(sets),
            "adjoint_ms": a[0] * 1e3, "adjoint_kernels_ms": a[1],
            "bump_ms": b[0] * 1e3, "bump_kernels_ms": b[1],
            "price_only_ms": one[0] * 1e3, "price_only_kernels_ms": one[1],
            "bump_one_dispatch_ms": m[0] * 1e3, "bump_one_dispatch_kernels_ms": m[1],
            "speedup": b[0] / a[0], "speedup_11x_one": len(sets) * one[0] / a[0],
            "speedup_vs_one_dispatch_bump": m[0] / a[0],
            "greeks_adjoint": [float(g) for g in a[2]], "greeks_bump": [float(g) for g in fd],
            "max_abs_diff": float(np.max(np.abs(fd - a[2]))),
            "one_dispatch_prices_equal": bool(np.array_equal(m[2], b[2])),
            "reference": "cpu-jit, 2M scenarios: adjoint 1.11 s vs 11 bump replays 10.76 s (9.7x), README.md:70-71"}


def host_cpu() -> dict:
    """The host's CPUs: the count the OS reports, the ones this process may
    run on, the thread budget the environment sets, and the model name."""
    model = None
    try:
        for line in Path("/proc/cpuinfo").read_text().splitlines():
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    usable = len(os.sched_getaffinity(0)) if hasattr(os, "sched_getaffinity") else (os.cpu_count() or 1)
    return {"nproc": os.cpu_count(), "usable": usable, "omp_num_threads": os.environ.get("OMP_NUM_THREADS"),
            "model": model}


def cpu_baseline(flat, sample, seed):
    sys.path.insert(0, str(ROOT / "oracle"))
    import oracle

    cpu = host_cpu()
    # Every CPU this process may use, unless the environment sets a smaller thread budget (a shared host
    # gives each GPU a share of its cores through OMP_NUM_THREADS).
    threads = cpu["usable"]
    if cpu["omp_num_threads"] and cpu["omp_num_threads"].isdigit():
        threads = min(threads, int(cpu["omp_num_threads"]))
    oracle.replay_sums(flat, 4096, 0, seed, threads=threads)  # load + warm
    t0 = time.perf_counter()
    oracle.replay_sums(flat, sample, 0, seed, threads=threads)
    secs = time.perf_counter() - t0
    return {"value": sample / secs, "unit": "scenarios/s", "cores": threads, "kind": "port", "host": cpu,
            "sample": f"{WORKLOAD}, fp64, {sample:,} scenarios, seed {seed}: C restatement of the reference "
                      f"scalar cpu engine (oracle/nt_oracle.c), OpenMP over {threads} threads, {secs:.2f} s; "
                      "reference cpu-jit/simd not run (no JDK on this host)"}


def copy_calibration(mib: int) -> int:
    import torch

    n = mib << 20
    a = torch.ones(n, dtype=torch.uint8, device="cuda")
    b = torch.empty_like(a)
    for _ in range(3):
        b.copy_(a)
    torch.cuda.synchronize()
    print(json.dumps({"copy_bytes": n, "copies": 3}), flush=True)
    return 0


def other_workload(rocm, args) -> int:
    from nablatensor_amd import workloads

    desc, paths, seed, prec = workloads.DESCRIPTIONS[args.workload]
    prec = args.precision or prec
    paths = args.paths if args.paths != 2_000_000 else paths
    flat = workload_tape(args.workload, args.coefficients)
    if args.workload == "local_vol":
        desc = f"{desc}, k = {args.coefficients}"
    if args.price_only:
        desc = f"{desc.split(', value')[0]}, value only"
    print(f"[bench] {args.workload} {desc}: {len(flat['op'])} nodes, {paths:,} scenarios/step, {prec}",
          file=sys.stderr, flush=True)
    if args.markets > 1 or args.price_only:
        m = measure_markets(rocm, flat, prec, paths, args.steps, args.warmup, seed, args.markets, args.ramp,
                            adjoints=not args.price_only)
        what = "value" if args.price_only else "value+all Greeks"
        out = {"metric": f"market-scenarios/sec for {what} ({prec}, {args.markets} input sets per dispatch)",
               "value": m["value"], "unit": "market-scenarios/s", "n_gpus": 1, "steps": args.steps,
               "warmup": args.warmup, "ms_per_step": m["ms_per_step"], "higher_is_better": True, "scaling": "weak",
               "vs_baseline": None, "dtype": "f64" if prec == "fp64" else "f32",
               "data": f"synthetic (Philox2x32-10 normals, seed {seed})",
               "config": {"workload": f"{args.workload}: {desc}", "scenarios_per_step": paths, "seed": seed,
                          "markets": args.markets},
               "replay_kernel_ms": m["replay_kernel_ms"], "single_market_kernel_ms": m["single_market_kernel_ms"],
               "speedup_vs_separate": m["speedup_vs_separate"], "mode": m["mode"]}
        print(json.dumps(out), flush=True)
        return 0
    m = measure(rocm, flat, prec, paths, args.steps, args.warmup, seed, args.policy, args.seg, args.mode, args.ramp,
                args.workload, args.waves, args.max_blocks, args.basis, args.roll, args.block)
    out = {"metric": f"scenarios/sec for value+all Greeks ({prec})", "value": m["value"], "unit": "scenarios/s",
           "n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "ms_per_step": m["ms_per_step"],
           "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f64" if prec == "fp64" else "f32", "data": f"synthetic (Philox2x32-10 normals, seed {seed})",
           "config": {"workload": f"{args.workload}: {desc}", "scenarios_per_step": paths, "seed": seed,
                      "nodes": len(flat["op"]), "inputs": len(flat["input_node"])},
           "roofline": m["roofline"], "kernel_ms": m["kernel_ms"], "replay_kernel_ms": m["replay_kernel_ms"],
           "kernel": m["kernel"]}
    print(json.dumps(out), flush=True)
    return 0


def risk_run(rocm, args) -> int:
    """The worst-of risk run: 10^4 launches of 10^6 scenarios each (fp32, seed
    42, launch k over scenarios [k 10^6, (k + 1) 10^6), so the Philox counter
    crosses 2^32 from launch 4,295 on), timed end to end on the host, raw sums
    added in launch order. Prints one JSON line with the total time, the
    throughput, the price and Greeks of the 10^10 scenarios and their standard
    errors."""
    import numpy as np

    from nablatensor_amd import workloads

    desc, per, seed, prec = workloads.DESCRIPTIONS["C5"]
    prec = args.precision or prec
    launches = args.risk_launches
    flat = workload_tape("C5")
    print(f"[bench] C5 risk run: {launches:,} launches x {per:,} scenarios, {prec}", file=sys.stderr, flush=True)
    with rocm.Executable(flat, rocm.options(prec)) as x:
        x.replay(per, 0, seed)  # load the module, clocks up
        total = None
        kernel_ms = 0.0
        t0 = time.perf_counter()
        for k in range(launches):
            sums, tm = x.replay(per, k * per, seed)
            total = sums if total is None else total + sums
            kernel_ms += tm["replay_ms"]
            if k % 1000 == 999:
                print(f"[bench] {k + 1:,} launches, {time.perf_counter() - t0:.1f} s", file=sys.stderr, flush=True)
        secs = time.perf_counter() - t0
    n = launches * per
    nin = len(flat["input_node"])
    mean = total / n
    var = np.maximum(mean[1] - mean[0] ** 2, 0.0)
    out = {"metric": f"scenarios/sec for value+all Greeks ({prec}), worst-of risk run end to end",
           "value": n / secs, "unit": "scenarios/s", "n_gpus": 1, "steps": launches, "warmup": 1,
           "ms_per_step": secs / launches * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f64" if prec == "fp64" else "f32", "data": f"synthetic (Philox2x32-10 normals, seed {seed})",
           "config": {"workload": f"C5: {desc}", "scenarios": n, "launches": launches, "scenarios_per_launch": per,
                      "offsets": "launch k at k x scenarios_per_launch"},
           "seconds": secs, "replay_kernel_seconds": kernel_ms / 1e3, "price": float(mean[0]),
           "price_stderr": float(np.sqrt(var / n)), "greeks": [float(g) for g in mean[2:2 + nin]]}
    print(json.dumps(out), flush=True)
    return 0


# The other benchmark configurations, reported beside the headline in the default run: the engine's default
# plan, each at the scenarios per dispatch its configuration names, fewer timed steps (these are
# reports, not the headline).
OTHER_WORKLOADS = (("C1", "fp64"), ("C3", "fp32"), ("C3", "fp64"), ("C4", "fp64"), ("C5", "fp32"), ("C5", "fp64"),
                   ("asian_weekdays", "fp64"))


def other_workloads(rocm, steps: int = 5, warmup: int = 1, ramp: float = 0.2) -> dict:
    from nablatensor_amd import workloads

    out = {}
    for name, prec in OTHER_WORKLOADS:
        desc, paths, seed, _ = workloads.DESCRIPTIONS[name]
        m = measure(rocm, workload_tape(name), prec, paths, steps, warmup, seed, 0, 0, 0, ramp, name)
        ex = m["roofline"]["executed_frac"]
        out[f"{name}_{prec}"] = {"workload": desc, "scenarios_per_step": paths, "seed": seed,
                                 "value": m["value"], "unit": "scenarios/s", "ms_per_step": m["ms_per_step"],
                                 "replay_kernel_ms": m["replay_kernel_ms"], "frac": m["roofline"]["frac"],
                                 "executed_frac": ex, "traffic": m["roofline"]["traffic"],
                                 "peak_tflops": m["roofline"]["peak"], "mode": m["kernel"]["mode"],
                                 "vgprs": m["kernel"]["vgprs"], "scratch_bytes": m["kernel"]["scratch_bytes"]}
        print(f"[bench] {name} {prec} {m['value']:.3e} scen/s, {100 * m['roofline']['frac']:.1f} % of peak",
              file=sys.stderr, flush=True)
    return out


def local_vol_modes(rocm, k: int = 24, steps: int = 5, warmup: int = 1, ramp: float = 0.2) -> dict:
    """Both derivative modes on the parametric local-volatility Asian (k
    coefficients, k + 3 inputs), the tape on which the cost model picks the
    reverse sweep: each mode's kernel time, roofline fraction and executed
    fraction, and the mode the engine picks by itself."""
    from nablatensor_amd import workloads

    desc, paths, seed, prec = workloads.DESCRIPTIONS["local_vol"]
    flat = workload_tape("local_vol", k)
    out = {"workload": f"{desc}, k = {k}", "inputs": len(flat["input_node"]), "scenarios_per_step": paths}
    for mode in (1, 2):
        m = measure(rocm, flat, prec, paths, steps, warmup, seed, 0, 0, mode, ramp, "local_vol")
        out[MODES[mode]] = {"value": m["value"], "replay_kernel_ms": m["replay_kernel_ms"],
                            "frac": m["roofline"]["frac"], "executed_frac": m["roofline"]["executed_frac"],
                            "vgprs": m["kernel"]["vgprs"], "scratch_bytes": m["kernel"]["scratch_bytes"]}
        out["cost_model"] = m["kernel"]["cost_model"]
    with rocm.Executable(flat, rocm.options(prec)) as x:
        out["picked"] = MODES[x.info()["mode"]]
    out["reverse_speedup"] = out["tangent"]["replay_kernel_ms"] / out["reverse"]["replay_kernel_ms"]
    print(f"[bench] local_vol k={k}: reverse {out['reverse']['replay_kernel_ms']:.3f} ms, tangent "
          f"{out['tangent']['replay_kernel_ms']:.3f} ms, engine picks {out['picked']}", file=sys.stderr, flush=True)
    return out


def host_overheads(rocm, args) -> int:
    """Host-path costs around the replay kernel on the Asian 252 tape, fp64:
    building an executable (lowering + hipRTC compile, or a code-object cache
    hit), the host time each dispatch adds to its kernels, and a chunked
    replaySafe request through the engine layer against the kernel-only rate.
    The reference's counterparts: the 0.5 s chunking with calibration probes
    (AbstractAadExecutable.java:100-159, RocmAadEngine.java:85) and
    synchronous null-stream dispatches (HipRuntime.java:40-43)."""
    import tempfile

    import nablatensor_amd as nt

    flat = workload_tape("C2")
    opts = rocm.options("fp64")
    saved = os.environ.get("NABLATENSOR_ROCM_CACHE")
    compile_s = {}
    try:
        with tempfile.TemporaryDirectory() as d:
            for label, cache in (("uncached", "off"), ("cache_miss", d), ("cache_hit", d)):
                os.environ["NABLATENSOR_ROCM_CACHE"] = cache
                t0 = time.perf_counter()
                with rocm.Executable(flat, opts) as x:
                    compile_s[label] = {"create_s": time.perf_counter() - t0,
                                        "compile_s": x.info()["compile_seconds"]}
    finally:
        if saved is None:
            os.environ.pop("NABLATENSOR_ROCM_CACHE", None)
        else:
            os.environ["NABLATENSOR_ROCM_CACHE"] = saved
    print(f"[bench] create: {compile_s}", file=sys.stderr, flush=True)

    dispatch = {}
    for name, paths in (("C1", 1_000_000), ("C2", 2_000_000)):
        with rocm.Executable(workload_tape(name), opts) as x:
            t_ramp = time.perf_counter()
            while time.perf_counter() - t_ramp < args.ramp:
                x.replay(paths, 0, args.seed)
            rows = []
            for k in range(max(args.steps, 5)):
                t0 = time.perf_counter()
                _, tm = x.replay(paths, k * paths, args.seed)
                rows.append((time.perf_counter() - t0, tm["kernel_ms"] / 1e3, tm["replay_ms"] / 1e3))
        n = len(rows)
        wall = sum(r[0] for r in rows) / n
        kernels = sum(r[1] for r in rows) / n
        dispatch[name] = {"paths": paths, "wall_ms": wall * 1e3, "kernels_ms": kernels * 1e3,
                          "replay_kernel_ms": sum(r[2] for r in rows) / n * 1e3,
                          "host_overhead_us": (wall - kernels) * 1e6}
        print(f"[bench] dispatch {name}: {dispatch[name]}", file=sys.stderr, flush=True)

    total = args.host_paths
    mc = (nt.MonteCarlo.of(nt.Products.asianCall()).market(nt.EquityMarket.atmOneYear())
          .steps(252).greeks().fp64().on("rocm").build())
    exe = mc.executable()
    t0 = time.perf_counter()
    exe.calibrate(args.seed)
    calib = time.perf_counter() - t0
    t0 = time.perf_counter()
    res = exe.replaySafe(total, args.seed)
    safe = time.perf_counter() - t0
    chunk = exe.measuredPathsPerSecond() * exe.maxChunkSeconds()
    mc.close()
    kernel_rate = dispatch["C2"]["paths"] / (dispatch["C2"]["kernels_ms"] / 1e3)
    out = {"metric": "scenarios/sec of a chunked replaySafe request (fp64), end to end on the host",
           "value": total / safe, "unit": "scenarios/s", "n_gpus": 1, "steps": 1, "warmup": 0,
           "ms_per_step": safe * 1e3, "higher_is_better": True, "scaling": "weak", "vs_baseline": None,
           "dtype": "f64", "data": f"synthetic (Philox2x32-10 normals, seed {args.seed})",
           "config": {"workload": f"{WORKLOAD}, replaySafe over {total:,} scenarios (0.5 s chunks)"},
           "replay_safe": {"paths": total, "seconds": safe, "chunk_paths_at_end": int(chunk),
                           "calibration_s": calib,
                           "vs_kernel_rate": total / safe / kernel_rate, "price": res.value()},
           "create": compile_s, "dispatch": dispatch}
    print(json.dumps(out), flush=True)
    return 0


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=20)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--ramp", type=float, default=0.5,
                    help="seconds of untimed replays before the warmup steps, so the GPU clocks are up")
    ap.add_argument("--paths", type=int, default=2_000_000)
    ap.add_argument("--seed", type=int, default=42)
    ap.add_argument("--policy", type=int, default=0, help="checkpoint policy (0 auto, 1 recompute, 2 store draws, 3 store all)")
    ap.add_argument("--seg", type=int, default=0, help="loop iterations per checkpoint segment (0 auto)")
    ap.add_argument("--mode", type=int, default=0, help="derivative mode (0 cost model, 1 reverse sweep, 2 tangent)")
    ap.add_argument("--max-blocks", type=int, default=0,
                    help="cap on the replay grid in blocks (0: the engine's own, whole blocks per CU, up to 8 resident grids)")
    ap.add_argument("--basis", type=int, default=0, choices=(0, 1, 2),
                    help="with --workload/--precision: tangent loops over 1 the inputs, 2 the loop's parameters "
                         "(0: the engine's choice)")
    ap.add_argument("--waves", type=int, default=0,
                    help="with --workload/--precision: minimum waves per SIMD asked of the compiler (0: the engine's choice)")
    ap.add_argument("--no-reverse", action="store_true", help="skip the reverse-sweep comparison run")
    ap.add_argument("--markets", type=int, default=1,
                    help="with --workload/--precision: price this many input sets per dispatch from shared draws")
    ap.add_argument("--price-only", action="store_true",
                    help="with --markets: price the input sets without Greeks")
    ap.add_argument("--cpu-sample", type=int, default=3_000_000,
                    help="scenarios in the CPU baseline's timed sample (about 25 CPU-seconds on 16 threads)")
    ap.add_argument("--no-fp32", action="store_true")
    ap.add_argument("--no-bump", action="store_true",
                    help="skip timing the adjoint against the 11 replays of a central bump-and-revalue")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--no-workloads", action="store_true",
                    help="skip the other benchmark configurations reported beside the headline")
    ap.add_argument("--coefficients", type=int, default=24,
                    help="with --workload local_vol: coefficients of the local-volatility polynomial")
    ap.add_argument("--workload", default="C2", choices=["C1", "C2", "C3", "C4", "C5", "asian_weekdays", "local_vol"],
                    help="C2 (default) prints the headline line; the others print the same fields for that workload")
    ap.add_argument("--precision", choices=["fp64", "fp32"], default=None,
                    help="run one workload at one precision and print its line (default: the workload's own; "
                         "for C2 without it, the headline line with fp64, the reverse sweep and fp32)")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="MIB",
                    help="only run a plain device-to-device copy of MIB MiB (3 times) and exit: the known-size "
                         "kernel that scales rocprofv3 FETCH_SIZE / WRITE_SIZE to bytes")
    ap.add_argument("--host", action="store_true",
                    help="only measure the host path around the kernel (executable creation with and without the "
                         "code-object cache, per-dispatch host time, a chunked replaySafe request) and print its line")
    ap.add_argument("--host-paths", type=int, default=4_000_000_000,
                    help="scenarios in the --host replaySafe request")
    ap.add_argument("--block", type=int, default=0,
                    help="threads per block (0: the engine's choice)")
    ap.add_argument("--roll", type=int, default=1, choices=(1, -1),
                    help="with --workload/--precision: -1 lowers the tape without its step loop (a checkpointed "
                         "straight line in reverse mode)")
    ap.add_argument("--risk-run", action="store_true",
                    help="only run the worst-of risk run (10^4 launches of 10^6 scenarios, fp32) and print its line")
    ap.add_argument("--risk-launches", type=int, default=10_000, help="launches in --risk-run")
    args = ap.parse_args()
    if args.copy_calibration:
        return copy_calibration(args.copy_calibration)
    if args.gpus != 1:
        print(f"bench.py measures one GPU only; --gpus {args.gpus} is not supported (scenarios shard by path "
              "range, each GPU returning its raw sums for one fixed-order reduction)", file=sys.stderr)
        return 2

    import nablatensor_amd as nt
    from nablatensor_amd import rocm

    if rocm.probe() < 1:
        print("no gfx950 device visible", file=sys.stderr)
        return 1
    if args.host:
        return host_overheads(rocm, args)
    if args.risk_run:
        return risk_run(rocm, args)
    if args.workload != "C2" or args.precision or args.markets > 1 or args.roll != 1:
        return other_workload(rocm, args)
    flat = nt.record(nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), nt.TimeGrid.uniform(252)).flat()
    print(f"[bench] {WORKLOAD}: {len(flat['op'])} nodes, {args.paths:,} scenarios/step", file=sys.stderr, flush=True)
    f64 = measure(rocm, flat, "fp64", args.paths, args.steps, args.warmup, args.seed, args.policy, args.seg,
                  args.mode, args.ramp)
    print(f"[bench] fp64 {f64['kernel']['mode']} {f64['value']:.3e} scen/s", file=sys.stderr, flush=True)
    rev = None
    if not args.no_reverse and f64["kernel"]["mode"] != "reverse":
        rev = measure(rocm, flat, "fp64", args.paths, args.steps, args.warmup, args.seed, args.policy, args.seg, 1,
                      args.ramp)
        print(f"[bench] fp64 reverse {rev['value']:.3e} scen/s", file=sys.stderr, flush=True)
    f32 = None
    if not args.no_fp32:
        f32 = measure(rocm, flat, "fp32", args.paths, args.steps, args.warmup, args.seed, args.policy, args.seg,
                      args.mode, args.ramp)
        print(f"[bench] fp32 {f32['kernel']['mode']} {f32['value']:.3e} scen/s", file=sys.stderr, flush=True)
    bump = None
    if not args.no_bump:
        bump = adjoint_vs_bump(rocm, flat, args.paths, args.seed)
        print(f"[bench] adjoint {bump['adjoint_ms']:.3f} ms vs 11 bump replays {bump['bump_ms']:.3f} ms "
              f"({bump['speedup']:.1f}x)", file=sys.stderr, flush=True)
    cpu = None if args.no_cpu_baseline else cpu_baseline(flat, args.cpu_sample, args.seed)
    others = None if args.no_workloads else other_workloads(rocm)
    modes = None if args.no_workloads else local_vol_modes(rocm)
    out = {
        "metric": "scenarios/sec for value+all Greeks (fp64), % of VALU FP64 peak",
        "value": f64["value"],
        "unit": "scenarios/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": f64["ms_per_step"],
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": f64["value"] / REFERENCE_ROCM_FP64,
        "baseline": "reference rocm engine fp64 on Radeon 780M (gfx1103), docs/examples/asian-greeks.md:43",
        "dtype": "f64",
        "data": "synthetic (Philox2x32-10 normals, seed 42)",
        "config": {"workload": WORKLOAD, "scenarios_per_step": args.paths, "seed": args.seed,
                   "nodes": len(flat["op"]), "steps": 252, "greeks": 5},
        "roofline": f64["roofline"],
        "kernel_ms": f64["kernel_ms"],
        "replay_kernel_ms": f64["replay_kernel_ms"],
        "kernel": f64["kernel"],
        "reverse": None if rev is None else {k: rev[k] for k in ("value", "ms_per_step", "replay_kernel_ms",
                                                                  "roofline", "kernel")},
        "fp32": None if f32 is None else {k: f32[k] for k in ("value", "ms_per_step", "replay_kernel_ms",
                                                               "roofline", "kernel")},
        "adjoint_vs_bump": bump,
        "cpu_baseline": cpu,
        "workloads": others,
        "local_vol_modes": modes,
    }
    print(json.dumps(out), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
