"""Shared fixtures: the five workload tapes, recorded by the host layer.

Tests marked `gpu` need an MI355X (gfx950) and the in-tree libnt_rocm.so;
everything else runs on the CPU. The oracle (oracle/oracle.py) is the checker.
"""
from __future__ import annotations

import json
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))
sys.path.insert(0, str(ROOT / "tests"))

GOLDEN = ROOT / "tests" / "golden"


def reference_values() -> dict:
    """Values held by the reference repository (tests/golden/reference_values.json)."""
    return json.loads((GOLDEN / "reference_values.json").read_text())


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) device and the built HIP engine")


@pytest.fixture(scope="session")
def nt():
    import nablatensor_amd
    return nablatensor_amd


def equity_tape(nt, product, market, steps):
    return nt.record(product, market, nt.TimeGrid.uniform(steps))


def workload_tapes(nt, steps_c4: int = 504, steps_c5: int = 252) -> dict:
    """Tapes of the five workloads (nablatensor_amd/workloads.py)."""
    from nablatensor_amd import workloads
    return workloads.workload_tapes(steps_c4, steps_c5)


@pytest.fixture(scope="session")
def tapes(nt):
    return {k: v.flat() for k, v in workload_tapes(nt).items()}


def tape_slots(source: str) -> int:
    for line in source.splitlines():
        if line.startswith("// nt-plan:"):
            for kv in line.split()[2:]:
                k, v = kv.split("=")
                if k == "tape_slots":
                    return int(v)
    raise ValueError("no plan line in the generated source")


def rel_err(a, b, floor: float = 1.0) -> float:
    """max |a-b| / max(floor, |b|) elementwise (the reference's 1+|x| style scale)."""
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    return float(np.max(np.abs(a - b) / np.maximum(floor, np.abs(b)))) if a.size else 0.0


def gpu_available() -> bool:
    try:
        from nablatensor_amd import rocm
        return rocm.probe() > 0
    except Exception:
        return False


COND_STRICT = 1e-5  # distance to a singular point at or above which a path must meet 1e-12


ILL_CONDITIONED_TOL = 1e-8


def per_path_bounds(cond: np.ndarray, tol: float = 1e-12) -> np.ndarray:
    """Per-path tolerance: `tol` on well-conditioned paths. A path that comes
    within 1e-5 of a singular point of an active node (SQRT/LOG argument, DIV
    denominator, MAX/MIN tie) amplifies a last-bit difference in its draws
    roughly as 1e-17 / distance (measured on the Heston tape, where the
    variance grazes the full-truncation floor); such paths are held to 1e-8."""
    return np.where(cond >= COND_STRICT, tol, ILL_CONDITIONED_TOL)


def check_per_path(values, grads, flat, paths, offset, seed, tol=1e-12, min_strict=0.5):
    """Compares per-path values/adjoints with the oracle (value componentwise,
    gradient normwise) under per_path_bounds; returns a summary dict."""
    import oracle
    ov, og = oracle.replay_paths(flat, paths, offset, seed)
    ev, eg = oracle.path_errors(values, grads, ov, og)
    sing, tie = oracle.conditioning(flat, paths, offset, seed)
    cond = np.minimum(sing, tie)
    bound = per_path_bounds(cond, tol)
    err = np.maximum(ev, eg)
    strict = cond >= COND_STRICT
    out = {"max_err_strict": float(err[strict].max()) if strict.any() else 0.0,
           "max_err_all": float(err.max()), "strict_paths": int(strict.sum()), "paths": paths,
           "violations": int(np.sum(err > bound))}
    assert out["violations"] == 0, out
    assert strict.mean() >= min_strict, out
    return out


def jump_clock_tape(nt, steps=16):
    """The reference's RandomStreamsTest body (RandomStreamsTest.java:70-84): a
    normal on the default stream and a uniform on a named stream per step; the
    smooth jump indicator 1 / (1 + exp(-(u - 0.97) / 0.01)) stands in for
    Smooth.gt."""
    def body(rec):
        s0 = rec.input("S0", 100.0)
        vol = rec.input("sigma", 0.2)
        jumps = rec.stream("jump-clock")
        acc = s0
        for _ in range(steps):
            z = rec.randn()
            u = jumps.randu()
            jump = u.sub(0.97).mul(-100.0).exp().add(1.0)
            jump = rec.constant(1.0).div(jump)
            acc = acc.mul(vol.mul(z).mul(0.05).add(1.0)).add(jump.mul(2.0))
        rec.output(acc)
    return nt.AadRecorder.record(body)


def two_output_tape(nt, steps=40):
    """Two outputs of one GBM path with a uniform-driven barrier shift: the
    terminal spot and the running maximum (MultiOutput-style measures)."""
    def body(rec):
        s0 = rec.input("S0", 100.0)
        vol = rec.input("sigma", 0.25)
        r = rec.input("r", 0.03)
        dt = 1.0 / steps
        drift = r.sub(vol.mul(vol).mul(0.5)).mul(dt)
        sd = vol.mul(dt ** 0.5)
        s = s0
        hi = s0
        for _ in range(steps):
            s = s.mul(drift.add(sd.mul(rec.randn())).exp())
            hi = hi.max(s.mul(rec.stream("shift").randu().mul(0.01).add(0.995)))
        rec.output("spot", s)
        rec.output("max", hi)
    return nt.AadRecorder.record(body)


def scaled_exp_tape(nt, a, steps=16):
    """s <- s exp(a z) per step: every exponent is a loop-invariant times a
    normal draw, so the kernel bounds it once per path (6.77 |a| <= 708)
    instead of checking each exponential; a = 300 fails that bound."""
    def body(rec):
        s0 = rec.input("S0", 1.0)
        k = rec.input("a", a)
        s = s0
        for _ in range(steps):
            s = s.mul(k.mul(rec.randn()).exp())
        rec.output(s)
    return nt.AadRecorder.record(body)


def sqrt_classes_tape(nt, s_val, floor=True, steps=16):
    """acc <- acc + w sqrt(x), x = max(z s, 0) (or z s without the floor): x
    is +0 for z <= 0 (the max follows its constant, so no derivative flows
    through the infinite factor of sqrt at 0) and subnormal for z > 0 when
    s = 1e-310; without the floor x < 0 gives a NaN root."""
    def body(rec):
        s = rec.input("s", s_val)
        w = rec.input("w", 1.0)
        acc = w.mul(0.0)
        for _ in range(steps):
            z = rec.randn()
            x = z.mul(s).max(0.0) if floor else z.mul(s)
            acc = acc.add(x.sqrt().mul(w))
        rec.output(acc)
    return nt.AadRecorder.record(body)
