"""bench.py's JSON contract, exercised on the CPU with the device measurements
replaced by fixed numbers (no GPU is touched)."""
from __future__ import annotations

import json
import sys

import pytest

import conftest

sys.path.insert(0, str(conftest.ROOT))
import bench  # noqa: E402

LOCAL_VOL_MODES = bench.local_vol_modes  # the real one: the fixture below replaces it for the headline tests


def fake_measure(rocm, flat, precision, paths, steps, warmup, seed, policy, seg, mode=0, ramp=0.5, workload="C2",
                 waves=0, max_blocks=0, basis=0, roll=1, block=0):
    ms = 2.0 if precision == "fp64" else 1.0
    resolved = "reverse" if mode == 1 else "tangent"
    return {"value": paths / (ms / 1e3), "ms_per_step": ms, "kernel_ms": ms, "replay_kernel_ms": ms,
            "kernel_scenarios_per_s": paths / (ms / 1e3),
            "roofline": {"bound": "valu", "kernel": "nt_replay", "achieved": 10.0, "peak": 78.6, "unit": "TFLOP/s",
                         "frac": 10.0 / 78.6, "traffic": None, "traffic_source": None, "algorithmic_bytes": 1,
                         "executed_flops_per_scenario": 15000, "executed_achieved": 8.0, "executed_frac": 8.0 / 78.6,
                         "valu_issue": 0.85, "executed_source": "fake",
                         "flops_per_scenario": 18723, "convention": "NT-FLOP v1"},
            "kernel": {"vgprs": 100, "scratch_bytes": 0, "mode": resolved,
                       "cost_model": {"forward": 1, "reverse": 2, "tangent": 3}}}


@pytest.fixture
def patched(monkeypatch):
    from nablatensor_amd import rocm

    monkeypatch.setattr(rocm, "probe", lambda: 1)
    monkeypatch.setattr(bench, "measure", fake_measure)
    monkeypatch.setattr(bench, "cpu_baseline", lambda flat, sample, seed: {
        "value": 1e6, "unit": "scenarios/s", "cores": 16, "kind": "port", "sample": "fake"})
    monkeypatch.setattr(bench, "local_vol_modes", lambda rocm: {"picked": "reverse", "reverse_speedup": 1.5})
    monkeypatch.setattr(bench, "adjoint_vs_bump", lambda rocm, flat, paths, seed: {"speedup": 10.0,
                                                                                   "adjoint_ms": 1.0,
                                                                                   "bump_ms": 10.0})


def run_main(monkeypatch, capsys, argv):
    monkeypatch.setattr(sys, "argv", ["bench.py", *argv])
    assert bench.main() == 0
    lines = [ln for ln in capsys.readouterr().out.splitlines() if ln.strip()]
    assert len(lines) == 1
    return json.loads(lines[0])


def test_headline_line_has_the_contract_fields(patched, monkeypatch, capsys):
    out = run_main(monkeypatch, capsys, ["--steps", "2", "--warmup", "1"])
    for key in ("metric", "value", "unit", "n_gpus", "steps", "warmup", "ms_per_step", "higher_is_better",
                "scaling", "vs_baseline", "dtype", "data", "config", "roofline", "cpu_baseline"):
        assert key in out, key
    assert out["n_gpus"] == 1 and out["steps"] == 2 and out["warmup"] == 1
    assert out["dtype"] == "f64" and out["higher_is_better"] is True
    assert out["vs_baseline"] == pytest.approx(out["value"] / bench.REFERENCE_ROCM_FP64)
    assert out["roofline"]["frac"] == pytest.approx(out["roofline"]["achieved"] / out["roofline"]["peak"])
    assert out["cpu_baseline"]["kind"] in ("port", "reference")
    assert out["reverse"]["kernel"]["mode"] == "reverse"
    assert out["fp32"]["value"] > 0
    assert out["adjoint_vs_bump"]["speedup"] == 10.0
    assert out["local_vol_modes"]["picked"] == "reverse"
    w = out["workloads"]
    assert set(w) == {"C1_fp64", "C3_fp32", "C3_fp64", "C4_fp64", "C5_fp32", "C5_fp64", "asian_weekdays_fp64"}
    assert all(r["value"] > 0 and 0 < r["frac"] < 1 for r in w.values())


@pytest.mark.parametrize("workload", ["C1", "C3", "C4", "C5"])
def test_other_workloads_print_one_line(patched, monkeypatch, capsys, workload):
    out = run_main(monkeypatch, capsys, ["--workload", workload, "--steps", "1", "--warmup", "0"])
    assert out["config"]["workload"].startswith(workload)
    assert out["value"] > 0


def test_measure_prices_the_roofline_from_the_replay_kernel_time(monkeypatch):
    """bench.measure with a stand-in executable on the Asian call's default
    plan: achieved = NT-FLOP per scenario x scenarios / the replay kernel's
    mean event time, frac = achieved / the fp64 peak, algorithmic bytes = the
    inputs plus one partial per channel and block, and traffic and executed
    FLOPs from the committed counter summary of that kernel."""
    import numpy as np

    from nablatensor_amd import rocm

    flat = bench.workload_tape("C2")

    class FakeExecutable:
        def __init__(self, flat, opts):
            self.n = len(flat["input_node"])

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

        def info(self):
            return {"vgprs": 84, "sgprs": 86, "scratch_bytes": 0, "lds_bytes": 18688, "loop_period": 6,
                    "loop_iters": 252, "seg_len": 2, "n_segments": 126, "checkpoint": 0, "tape_slots": 0,
                    "grid_cap": 10240, "mode": 2}

        def grid(self, paths):
            return 4096, 256

        def source(self):
            return "// nt-cost: forward=13656 reverse=16688 tangent=4586\n"

        def replay(self, paths, offset, seed):
            return np.zeros(2 + self.n), {"kernel_ms": 0.81, "wall_ms": 0.85, "replay_ms": 0.8}

    monkeypatch.setattr(rocm, "Executable", FakeExecutable)
    out = bench.measure(rocm, flat, "fp64", 2_000_000, 3, 1, 42, 0, 0, ramp=0.0, workload="C2")
    r = out["roofline"]
    assert out["replay_kernel_ms"] == pytest.approx(0.8) and out["kernel_ms"] == pytest.approx(0.81)
    assert r["flops_per_scenario"] == 18_723 and r["peak"] == 78.6
    assert r["achieved"] == pytest.approx(18_723 * 2e6 / 0.8e-3 / 1e12)
    assert r["frac"] == pytest.approx(r["achieved"] / 78.6)
    assert r["algorithmic_bytes"] == 8 * (5 + 4096 * 7)
    assert r["traffic"] is not None and r["traffic_source"].endswith("nt_replay_asian252_fp64_counters.md")
    assert r["executed_flops_per_scenario"] > 0
    assert r["executed_frac"] == pytest.approx(r["executed_flops_per_scenario"] * 2e6 / 0.8e-3 / 1e12 / 78.6)
    assert out["kernel"]["grid"] == 4096 and out["kernel"]["mode"] == "tangent"


def test_risk_run_line(patched, monkeypatch, capsys):
    """--risk-run adds the raw sums of every launch (launch k over scenarios
    k x 10^6 onwards) and reports the time and the 10^10-scenario result."""
    import numpy as np

    from nablatensor_amd import rocm

    offsets = []

    class FakeExecutable:
        def __init__(self, flat, opts):
            self.n = len(flat["input_node"])

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

        def replay(self, paths, offset, seed):
            offsets.append(offset)
            sums = np.zeros(2 + self.n)
            sums[0], sums[1] = 2.0 * paths, 5.0 * paths
            return sums, {"kernel_ms": 1.0, "wall_ms": 1.0, "replay_ms": 1.0}

    monkeypatch.setattr(rocm, "Executable", FakeExecutable)
    out = run_main(monkeypatch, capsys, ["--risk-run", "--risk-launches", "3"])
    assert offsets == [0, 0, 1_000_000, 2_000_000]
    assert out["config"]["scenarios"] == 3_000_000 and out["steps"] == 3
    assert out["price"] == 2.0 and out["price_stderr"] == pytest.approx(1.0 / np.sqrt(3e6))
    assert out["dtype"] == "f32" and len(out["greeks"]) == 33


def test_more_than_one_gpu_is_refused(monkeypatch, capsys):
    monkeypatch.setattr(sys, "argv", ["bench.py", "--gpus", "8"])
    assert bench.main() == 2
    assert "one GPU" in capsys.readouterr().err


def test_markets_line(patched, monkeypatch, capsys):
    monkeypatch.setattr(bench, "measure_markets", lambda *a, **k: {
        "value": 1e9, "ms_per_step": 2.0, "replay_kernel_ms": 2.0, "single_market_kernel_ms": 1.0, "markets": 4,
        "mode": "tangent", "speedup_vs_separate": 2.0})
    out = run_main(monkeypatch, capsys, ["--workload", "C2", "--markets", "4", "--steps", "1", "--warmup", "0"])
    assert out["unit"] == "market-scenarios/s" and out["config"]["markets"] == 4


COUNTED = [("C2", "fp64", 0, 1), ("C2", "fp64", 1, 1), ("C2", "fp32", 0, 1), ("C2", "fp64", 1, -1),
           *[(w, p, 0, 1) for w, p in bench.OTHER_WORKLOADS], ("local_vol", "fp64", 0, 1), ("local_vol", "fp64", 2, 1)]


@pytest.mark.parametrize("workload,precision,mode,roll", COUNTED)
def test_committed_counters_cover_the_planned_kernels(workload, precision, mode, roll):
    """The traffic and executed-FLOP figures bench.py reports come from the
    committed rocprofv3 summary of the exact kernel the engine builds today
    (derivative mode, checkpoint policy, segment length, segments, VGPRs from
    the compiled code object); a change of plan or of register allocation
    that leaves a reported kernel unmeasured fails here rather than printing
    null."""
    from nablatensor_amd import rocm

    info = rocm.compile_check(bench.workload_tape(workload), rocm.options(precision, mode=mode, roll=roll))
    got = bench.measured_counters(workload, precision, info)
    assert set(got) == {"traffic", "executed"}, (workload, precision, info)
    assert got["traffic"]["bytes"] > 0 and got["executed"]["flops_per_scenario"] > 0


@pytest.mark.gpu
@pytest.mark.parametrize("workload,precision,mode,roll", COUNTED)
def test_committed_counters_match_the_launch_grid(workload, precision, mode, roll):
    """On the device, the committed counter lines of each reported kernel were
    taken at the grid the engine launches today for the workload's scenarios
    per dispatch (the grid sets the partial rows, the HBM bytes and the
    tail), so a change of launch geometry that leaves the reported traffic
    stale fails here."""
    from nablatensor_amd import rocm, workloads

    paths = workloads.DESCRIPTIONS[workload][1]
    print(f"case {workload} {precision} mode={mode} roll={roll} paths={paths}", flush=True)
    with rocm.Executable(bench.workload_tape(workload), rocm.options(precision, mode=mode, roll=roll)) as x:
        info = x.info()
        grid, block = x.grid(paths)
    assert block == info["block"] and 1 <= grid <= info["grid_cap"]
    got = bench.measured_counters(workload, precision, info, grid)
    assert set(got) == {"traffic", "executed"}, (workload, precision, grid, info)


def test_adjoint_vs_bump_prices_the_eleven_sets(monkeypatch):
    """The bump leg replays the base market and +h, -h per input (price-only,
    the same paths and seed), takes central differences, and divides the 11
    replays' wall time by the adjoint dispatch's. A fake executable whose price
    is linear in the inputs (slope j + 1 for input j) and whose adjoint
    dispatch returns those slopes gives bump Greeks equal to them."""
    import numpy as np

    from nablatensor_amd import rocm

    slopes = np.arange(1.0, 6.0)

    class FakeExecutable:
        def __init__(self, flat, opts):
            self.adjoints = bool(opts.adjoints)
            self.x = np.array(flat["recorded_inputs"], dtype=float)

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

        def set_inputs(self, x):
            self.x = np.array(x, dtype=float)

        def _sums(self, x, paths):
            grads = slopes * paths if self.adjoints else np.zeros(5)
            return np.concatenate([[float(slopes @ x) * paths, 0.0], grads])

        def replay(self, paths, offset, seed):
            return self._sums(self.x, paths), {"kernel_ms": 1.0, "wall_ms": 1.0, "replay_ms": 1.0}

        def replay_many(self, sets, paths, offset, seed):
            return np.stack([self._sums(x, paths) for x in sets]), {"kernel_ms": 2.0, "wall_ms": 2.0,
                                                                    "replay_ms": 2.0}

    monkeypatch.setattr(rocm, "Executable", FakeExecutable)
    flat = {"recorded_inputs": [100.0, 100.0, 0.2, 0.03, 1.0]}
    out = bench.adjoint_vs_bump(rocm, flat, 1000, 42, ramp=0.0)
    assert out["replays"] == 11
    assert np.allclose(out["greeks_bump"], slopes, rtol=1e-9)
    assert np.allclose(out["greeks_adjoint"], slopes)
    assert out["bump_kernels_ms"] == 11.0 and out["adjoint_kernels_ms"] == 1.0
    assert out["speedup"] == pytest.approx(out["bump_ms"] / out["adjoint_ms"])
    assert out["one_dispatch_prices_equal"] is True


def test_local_vol_modes_reports_both_sweeps(patched, monkeypatch):
    """The local-volatility row times the reverse sweep and tangent mode of
    the same tape and names the mode the engine picks on its own."""
    from nablatensor_amd import rocm

    class FakeExecutable:
        def __init__(self, flat, opts):
            pass

        def __enter__(self):
            return self

        def __exit__(self, *exc):
            return False

        def info(self):
            return {"mode": 1}

    monkeypatch.setattr(rocm, "Executable", FakeExecutable)
    out = LOCAL_VOL_MODES(rocm, k=4)
    assert out["inputs"] == 7 and out["picked"] == "reverse"
    assert out["reverse"]["replay_kernel_ms"] == 2.0 and out["tangent"]["replay_kernel_ms"] == 2.0
    assert out["reverse_speedup"] == 1.0 and out["cost_model"]["reverse"] == 2
