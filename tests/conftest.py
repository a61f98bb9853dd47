"""Shared fixtures: the five workload tapes, recorded by the host layer.

Tests marked `gpu` need an MI355X (gfx950) and the in-tree libnt_rocm.so;
everything else runs on the CPU. Results are held to the oracle (oracle/oracle.py).
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


# Per-path bar. Each path is held, per component (its value and each
# derivative, relative with floor 1), to max(TOL, SENS_K x s), where s is the
# oracle's own sensitivity: the largest change of that component when the
# oracle replays the path with every transcendental result moved by one unit
# (log, sqrt, exp by one ulp; Box-Muller's sin and cos by 2^-53), up or down in
# each of the fixed pseudo-random patterns SENS_PATTERNS. A correct engine
# differs from the oracle by last-place differences of its libm (the
# skeleton's own log within 2 ulp, sin/cos within 2 * 2^-53) and of its
# arithmetic order; a well-conditioned path has s below TOL / SENS_K and is held
# to TOL. Measured on the CPU emulation of the kernels (4,096 Heston paths,
# both derivative modes): actual error / s has median 0.4, and no component
# above 1e-12 exceeds 4 s; SENS_K = 8 keeps a factor 2 beyond that.
TOL = 1e-12
SENS_K = 8.0
SENS_PATTERNS = (1, 2, 3)
# Fraction of paths held to TOL on every component, per workload: the lowest
# measured over the path samples the tests use (30 to 4,096 paths at offset
# 0x100000003, seeds 42 and 7). The rest are paths whose value is a small
# difference of large quantities (an Asian or barrier payoff just in the
# money: A - K with A near 100 loses two digits against the floor of 1) or,
# in the Heston tape, whose variance grazes the full-truncation floor.
STRICT = {"C1": 1.0, "C2": 0.94, "C3": 0.84, "C4": 0.80, "C5": 0.95}
# Fraction of paths allowed above TOL on some component, per workload: the
# count measured on MI355X with about 1.5x margin (C3: 1 of 1,024 paths;
# C4: 30 of 4,096 and 3 of 512; none on C1, C2, C5 and the other tapes).
ABOVE = {"C1": 0.0, "C2": 0.001, "C3": 0.002, "C4": 0.01, "C5": 0.004}
# Error over sensitivity on the components held to SENS_K x s: measured on
# MI355X (every per-path test, both modes) at most 1.53 at the 99th percentile
# and 2.92 at the maximum; these bars keep a regression that stays inside
# SENS_K x s from passing unseen.
RATIO_P99 = 2.0
RATIO_MAX = 4.0


def componentwise_errors(values, grads, ref_values, ref_grads):
    """Per path: |dv| / max(1, |v|), and per derivative |dg_j| / max(1, |g_j|).
    Equal values (also equal infinities) and NaN against NaN agree; any other
    non-finite difference is an infinite error."""
    def rel(a, b):
        a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
        with np.errstate(invalid="ignore"):
            d = np.abs(a - b)
            d = np.where((a == b) | (np.isnan(a) & np.isnan(b)), 0.0, d)
            d = np.where(np.isnan(d), np.inf, d)
            return d / np.maximum(1.0, np.nan_to_num(np.abs(b), nan=1.0))
    return rel(values, ref_values), rel(grads, ref_grads)


def path_sensitivity(flat, paths, offset, seed, inputs=None):
    """The oracle's per-path rows (values, gradients) and their sensitivity to
    one-unit moves of every transcendental result (same shapes), the largest
    over SENS_PATTERNS."""
    import oracle
    ov, og = oracle.replay_paths(flat, paths, offset, seed, inputs=inputs)
    sv, sg = np.zeros_like(ov), np.zeros_like(og)
    for pattern in SENS_PATTERNS:
        pv, pg = oracle.replay_paths(flat, paths, offset, seed, inputs=inputs, perturb=pattern)
        dv, dg = componentwise_errors(pv, pg, ov, og)
        sv, sg = np.maximum(sv, dv), np.maximum(sg, dg)
    return ov, og, sv, sg


def check_per_path(values, grads, flat, paths, offset, seed, tol=TOL, min_strict=1.0, inputs=None,
                   max_above=0.002):
    """Compares per-path values and derivatives with the oracle, component by
    component, under the sensitivity-scaled bound above. `min_strict` is the
    fraction of paths that must be held to `tol` on every component (their
    sensitivity is below tol / SENS_K), set at the measured fraction of the
    call's path sample: the fraction is a property of the oracle alone, and
    pinning it keeps the sensitivity measurement from excusing paths it did
    not excuse when the bar was set. At most `max_above` of the paths (rounded
    up) may exceed `tol` on any component, and on the components held to SENS_K x s
    the error over s stays within RATIO_P99 at the 99th percentile and
    RATIO_MAX at the worst. Returns a summary, with the normwise gradient
    error (max_j |dg_j| / max(1, max_j |g_j|)) beside."""
    import oracle
    ov, og, sv, sg = path_sensitivity(flat, paths, offset, seed, inputs)
    ev, eg = componentwise_errors(values, grads, ov, og)
    bv, bg = np.maximum(tol, SENS_K * sv), np.maximum(tol, SENS_K * sg)
    bad = (ev > bv) | (np.any(eg > bg, axis=1) if eg.size else False)
    strict = (bv == tol) & (np.all(bg == tol, axis=1) if bg.size else True)
    err = np.maximum(ev, eg.max(axis=1)) if eg.size else ev
    _, normwise = oracle.path_errors(values, grads, ov, og)
    # error over sensitivity on the components held to SENS_K x s rather than tol
    e_all = np.concatenate([ev.ravel(), eg.ravel()])
    s_all = np.concatenate([sv.ravel(), sg.ravel()])
    loose = SENS_K * s_all > tol
    ratio = e_all[loose] / s_all[loose]
    out = {"paths": paths, "violations": int(np.sum(bad)), "strict_fraction": float(np.mean(strict)),
           "paths_above_tol": int(np.sum(err > tol)), "max_err": float(err.max()),
           "max_err_strict": float(err[strict].max()) if strict.any() else 0.0,
           "max_normwise": float(normwise.max()) if normwise.size else 0.0,
           "loose_components": int(loose.sum()),
           "ratio_p99": float(np.percentile(ratio, 99)) if ratio.size else 0.0,
           "ratio_max": float(ratio.max()) if ratio.size else 0.0}
    assert out["violations"] == 0, out
    assert out["strict_fraction"] >= min_strict, out
    assert out["paths_above_tol"] <= int(np.ceil(max_above * paths)), out
    assert out["ratio_p99"] <= RATIO_P99 and out["ratio_max"] <= RATIO_MAX, out
    return out


def reconcile(got_sums, want_sums, paths, flat, seed, offset=0, sample=20_000, rel=1e-5, in_se=0.0):
    """fp32 against fp64 aggregates: the price and each Greek within `rel`
    relative, and `rel` normwise. `in_se` > 0 would let a Greek off at
    in_se x se_j instead, se_j its own Monte-Carlo standard error at `paths`
    scenarios (from the oracle's per-path rows of the first `sample` paths);
    no test uses it, and `within_se_floor` lists the Greeks above `rel` that
    0.05 se_j would have excused (a worst-of path whose two lowest assets end
    within fp32 rounding of each other credits its delta and vega to the other
    one, about 1 / n of a per-path Greek in absolute terms, which can exceed
    1e-5 of a small mean). Returns the per-Greek relative errors, the errors in
    standard errors, those Greeks, the normwise error max_j |dg_j| / max_j
    |g_j|, and `ok`."""
    import oracle
    got, want = oracle.to_result(got_sums, paths), oracle.to_result(want_sums, paths)
    _, rows = oracle.replay_paths(flat, min(paths, sample), offset, seed)
    se = rows.std(axis=0, ddof=1) / np.sqrt(paths)
    g, w = np.asarray(got["gradient"]), np.asarray(want["gradient"])
    d = np.abs(g - w)
    rel_err = d / np.abs(w)
    in_se_err = d / se
    by_floor = [int(j) for j in np.nonzero((rel_err > rel) & (in_se_err <= 0.05))[0]]
    out = {"price": abs(got["price"] - want["price"]) / abs(want["price"]),
           "greek_rel_max": float(rel_err.max()), "greek_worst": int(np.argmax(rel_err)),
           "greek_se_max": float(in_se_err.max()), "within_se_floor": by_floor,
           "normwise": float(d.max() / np.abs(w).max())}
    out["ok"] = bool(out["price"] <= rel and np.all(d <= np.maximum(rel * np.abs(w), in_se * se))
                     and out["normwise"] <= rel)
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


def no_input_tape(nt, steps=16):
    """A price with no inputs, so no Greeks: an Asian call on a GBM spot whose
    start, volatility and strike are literals (the sums are Σy and Σy² alone)."""
    def body(rec):
        s = rec.randn().mul(0.05).exp().mul(100.0)
        acc = s
        for _ in range(steps - 1):
            s = s.mul(rec.randn().mul(0.05).exp())
            acc = acc.add(s)
        rec.output(acc.mul(1.0 / steps).sub(100.0).max(0.0))
    return nt.AadRecorder.record(body)


def degenerate_tapes(nt):
    """Tapes at the edges of the format: no draws at all, an output that is an
    input node, an output with a zero derivative, and an output that is a
    draw (no active path to the inputs)."""
    def no_draws(rec):
        x, y = rec.input("x", 1.5), rec.input("y", 2.0)
        rec.output(x.mul(y).add(x.exp()))

    def input_out(rec):
        x, _ = rec.input("x", 1.5), rec.input("y", 2.0)
        rec.output(x)

    def const_out(rec):
        x = rec.input("x", 1.5)
        rec.output(x.mul(0.0).add(3.0))

    def draw_out(rec):
        rec.input("x", 1.5)
        rec.output(rec.randn())
    return {name: nt.AadRecorder.record(body).flat()
            for name, body in [("no_draws", no_draws), ("input_out", input_out), ("const_out", const_out),
                               ("draw_out", draw_out)]}


def branching_tape(nt, steps=24):
    """The reference's random branching tape for its checkpoint parity test
    (CudaCheckpointParityTest.java:75-85): a level driven by two normals per
    step and floored at 0.01, then log, exp, sqrt and a division."""
    def body(rec):
        level = rec.input("level", 1.2)
        scale = rec.input("scale", 0.1)
        for _ in range(steps):
            level = level.add(rec.randn().mul(scale)).add(rec.randn().mul(0.01)).max(0.01)
        rec.output(level.log().exp().sqrt().div(scale.add(1.0)))
    return nt.AadRecorder.record(body)


def random_tape(nt, seed: int, steps: int, outputs: int = 2):
    """A tape of random shape: two inputs, normals on two streams, uniforms,
    every operation, and one or two outputs."""
    rng = np.random.default_rng(seed)

    def body(rec):
        x = rec.input("x", 1.0 + rng.random())
        y = rec.input("y", 0.5 + rng.random())
        other = rec.stream("other")
        vals = [x, y]
        for _ in range(steps):
            a = vals[rng.integers(len(vals))]
            b = vals[rng.integers(len(vals))]
            k = rng.integers(12)
            if k == 0:
                v = a.add(rec.randn())
            elif k == 1:
                v = a.mul(other.randn())
            elif k == 2:
                v = a.sub(other.randu())
            elif k == 3:
                v = a.add(b)
            elif k == 4:
                v = a.mul(b)
            elif k == 5:
                v = a.div(b.abs().add(1.0))
            elif k == 6:
                v = a.mul(0.1).exp()
            elif k == 7:
                v = a.abs().add(1.0).log()
            elif k == 8:
                v = a.abs().sqrt()
            elif k == 9:
                v = a.max(b)
            elif k == 10:
                v = a.min(b).neg()
            else:
                v = a.sub(b.mul(0.5))
            vals.append(v)
        rec.output("first", vals[-1].add(vals[len(vals) // 3]))
        if outputs > 1:
            rec.output("second", vals[-2].add(vals[len(vals) // 2]))
    return nt.AadRecorder.record(body)


def asian_tape(nt, steps):
    """Products.asianCall on the ATM one-year market over `steps` uniform fixings."""
    return nt.record(nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), nt.TimeGrid.uniform(steps))


MERTON_FIELDS = ("spot", "strike", "vol", "rate", "maturity", "jumpIntensity", "jumpMean", "jumpVol")


def merton_call_tape(nt, market: dict, maturity=1.0, steps=128, width=2.0e-4):
    """MertonJumpModel.european(CALL, maturity, steps, width) as the reference
    records it (MertonJumpModel.java:59-121): the MertonJumpMarket inputs in
    field order (MertonJumpMarket.java, recorded up front by Nabla.Inputs,
    Nabla.java:201-207), kappa = exp(muJ + deltaJ^2/2) - 1 once, then per step
    a diffusion normal, a uniform and a jump normal (in that order), the
    compensator -ln(1 + lambda kappa dt), the log-Euler diffusion, the smoothed
    indicator Smooth.lt(u, lambda dt) = 1 / (1 + exp(-(lambda dt - u) / width))
    (Smooth.java:44-68) and the jump factor exp(muJ + deltaJ zJ) - 1; payoff
    max(S - K, 0) exp(-r T)."""
    dt = maturity / steps
    sqrt_dt = dt ** 0.5

    def body(rec):
        x = {f: rec.input(f, float(market[f])) for f in MERTON_FIELDS}
        rate, vol, lam, mu_j, dl_j = x["rate"], x["vol"], x["jumpIntensity"], x["jumpMean"], x["jumpVol"]
        kappa = mu_j.add(dl_j.mul(dl_j).mul(0.5)).exp().sub(1.0)
        s = x["spot"]
        for _ in range(steps):
            z = rec.randn()
            u = rec.randu()
            zj = rec.randn()
            compensator = lam.mul(kappa).mul(dt).add(1.0).log()
            drift = rate.sub(vol.mul(vol).mul(0.5)).mul(dt).sub(compensator)
            diffused = s.mul(drift.add(vol.mul(sqrt_dt).mul(z)).exp())
            p = lam.mul(dt)
            e = p.sub(u).div(width).neg().exp()
            occurs = rec.constant(1.0).div(e.add(1.0))
            factor = mu_j.add(dl_j.mul(zj)).exp().sub(1.0)
            s = diffused.mul(rec.constant(1.0).add(occurs.mul(factor)))
        intrinsic = s.sub(x["strike"]).max(0.0)
        discount = rate.neg().mul(maturity).exp()
        rec.output(intrinsic.mul(discount))
    return nt.AadRecorder.record(body)


def merton_series_call(spot, strike, maturity, rate, vol, lam, mu_j, dl_j):
    """The Merton jump-diffusion call as its truncated Poisson series of
    Black-Scholes prices (MertonJumpDiffusion.price, MertonJumpDiffusion.java:
    price(); Merton 1976): with kappa = exp(muJ + deltaJ^2/2) - 1 and
    lambda' = lambda (1 + kappa), the sum over n of Poisson(lambda' T) weights
    times Black-Scholes with sigma_n^2 = sigma^2 + n deltaJ^2 / T and
    r_n = r - lambda kappa + n ln(1 + kappa) / T (carry b = r_n), stopped once
    the weights cover 1 - 1e-14."""
    from math import erfc, exp, log, log1p, sqrt

    def ncdf(x):
        return 0.5 * erfc(-x / sqrt(2.0))

    def bs_call(r, b, sigma):
        d1 = (log(spot / strike) + (b + 0.5 * sigma * sigma) * maturity) / (sigma * sqrt(maturity))
        d2 = d1 - sigma * sqrt(maturity)
        return spot * exp((b - r) * maturity) * ncdf(d1) - strike * exp(-r * maturity) * ncdf(d2)

    kappa = exp(mu_j + 0.5 * dl_j * dl_j) - 1.0
    lam_t = lam * (1.0 + kappa) * maturity
    total, weight, covered = 0.0, exp(-lam_t), 0.0
    for n in range(256):
        sigma_n = sqrt(vol * vol + n * dl_j * dl_j / maturity)
        r_n = rate - lam * kappa + n * log1p(kappa) / maturity
        total += weight * bs_call(r_n, r_n, sigma_n)
        covered += weight
        if covered > 1.0 - 1e-14 and n > 0:
            break
        weight *= lam_t / (n + 1)
    return total


def discounted_weekday_asian_tape(nt, fixings: int = 252):
    """An Asian call on a weekday grid, each fixing discounted by a bank account
    that grows by exp(r dt_i) per step (a deterministic factor from the step
    schedule, read by the average every step): S_i / B_i averaged, minus the
    strike, floored at zero."""
    from nablatensor_amd import workloads
    times = workloads.weekday_fixings(fixings)

    def body(rec):
        s = rec.input("S0", 100.0)
        k = rec.input("K", 100.0)
        vol = rec.input("sigma", 0.2)
        r = rec.input("r", 0.03)
        t_mat = rec.input("T", 1.0)
        b = r.mul(0.0).add(1.0)
        acc = r.mul(0.0)
        prev = 0.0
        for t in times:
            dt = t_mat.mul(t - prev)
            prev = t
            s = s.mul(r.sub(vol.mul(vol).mul(0.5)).mul(dt).add(vol.mul(dt.sqrt()).mul(rec.randn())).exp())
            b = b.mul(r.mul(dt).exp())
            acc = acc.add(s.div(b))
        rec.output(acc.mul(1.0 / fixings).sub(k).max(rec.constant(0.0)))
    return nt.AadRecorder.record(body).flat()


def signed_basket_tape(nt, steps=40):
    """Three GBM spots read only by the payoff, each step's exponent in one of
    the signed affine forms of a draw: p - r w (w = 0.6 z1 + 0.8 z2, a
    correlated normal), r z1 - p and r z2 alone, with p and r computed from
    the inputs before the steps; payoff max(a + b + c - K, 0)."""
    dt = 1.0 / steps

    def body(rec):
        sa, sb, sc = rec.input("Sa", 100.0), rec.input("Sb", 90.0), rec.input("Sc", 110.0)
        va, vb, vc = rec.input("sa", 0.2), rec.input("sb", 0.3), rec.input("sc", 0.25)
        rate = rec.input("r", 0.03)
        pa = rate.sub(va.mul(va).mul(0.5)).mul(dt)
        ra = va.mul(dt ** 0.5)
        pb = vb.mul(vb).mul(0.5).sub(rate).mul(dt)
        rb = vb.mul(dt ** 0.5)
        rc = vc.mul(dt ** 0.5)
        a, b, c = sa, sb, sc
        for _ in range(steps):
            z1 = rec.randn()
            z2 = rec.randn()
            w = z1.mul(0.6).add(z2.mul(0.8))
            a = a.mul(pa.sub(ra.mul(w)).exp())
            b = b.mul(rb.mul(z1).sub(pb).exp())
            c = c.mul(rc.mul(z2).exp())
        rec.output(a.add(b).add(c).sub(300.0).max(rec.constant(0.0)))
    return nt.AadRecorder.record(body).flat()


MAX_MIN_OUTPUTS = 6


def max_min_tape(nt, only=None):
    """MAX and MIN of two inputs and of an input and a literal, each its own
    output (or output `only` alone, for the reverse sweep, which follows one
    output), for the edge cases of java.lang.Math.max/min (signed zeros, NaN,
    infinities)."""
    def body(rec):
        x = rec.input("x", 1.0)
        y = rec.input("y", 2.0)
        outs = [("max", lambda: x.max(y)), ("min", lambda: x.min(y)), ("max0", lambda: x.max(0.0)),
                ("min0", lambda: x.min(0.0)), ("maxm1", lambda: y.max(-1.0)),
                ("minmax", lambda: x.max(y).min(y.mul(2.0)))]
        for k, (name, f) in enumerate(outs):
            if only is None or only == k:
                rec.output(name, f())
    return nt.AadRecorder.record(body)


MAX_MIN_CASES = [(-0.0, 0.0), (0.0, -0.0), (-0.0, -0.0), (float("nan"), 1.0), (1.0, float("nan")),
                 (float("inf"), 1.0), (float("-inf"), 1.0), (float("-inf"), float("-inf")),
                 (float("inf"), float("-inf")), (2.0, 3.0), (-0.0, 5.0), (5.0, -0.0), (-3.0, -0.0)]


def same_special(a, b):
    """Equal as Math.max/min results: NaN where the other is NaN, otherwise
    equal values with equal signs of zero."""
    a, b = np.asarray(a), np.asarray(b)
    return bool(np.array_equal(np.isnan(a), np.isnan(b)) and
                np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)]) and
                np.array_equal(np.signbit(a[~np.isnan(a)]), np.signbit(b[~np.isnan(b)])))


SPECIAL_OUTPUTS = 8


def special_ops_tape(nt, only=None):
    """EXP, LOG, SQRT, DIV (and 1 / x, the literal-numerator reciprocal), ABS,
    NEG and MUL of inputs set to special values, each its own output (or
    output `only` alone, for the reverse sweep)."""
    def body(rec):
        x = rec.input("x", 1.0)
        y = rec.input("y", 2.0)
        outs = [("exp", lambda: x.exp()), ("log", lambda: x.log()), ("sqrt", lambda: x.sqrt()),
                ("div", lambda: x.div(y)), ("recip", lambda: rec.constant(1.0).div(x)), ("abs", lambda: x.abs()),
                ("neg", lambda: x.neg()), ("mul", lambda: x.mul(y))]
        for k, (name, f) in enumerate(outs):
            if only is None or only == k:
                rec.output(name, f())
    return nt.AadRecorder.record(body)


SPECIAL_CASES = [(-0.0, 1.0), (0.0, 1.0), (float("inf"), 1.0), (float("-inf"), 1.0), (float("nan"), 1.0),
                 (5e-324, 1.0), (-2.0, 1.0), (710.0, 2.0), (-746.0, 0.5), (1e308, 1e-308), (0.0, 0.0),
                 (1e-310, 3.0), (-1e-310, -3.0), (0.75, -0.0)]


def close_special(a, b, rel):
    """NaN where the other is NaN, the same infinities and signed zeros, and
    finite non-zero values within `rel` relative."""
    a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
    if not np.array_equal(np.isnan(a), np.isnan(b)):
        return False
    m = ~np.isnan(a)
    a, b = a[m], b[m]
    if not (np.array_equal(np.isinf(a), np.isinf(b)) and np.array_equal(a[np.isinf(a)], b[np.isinf(b)])):
        return False
    z = (a == 0) | (b == 0)
    if not (np.array_equal(a[z], b[z]) and np.array_equal(np.signbit(a[z]), np.signbit(b[z]))):
        return False
    f = np.isfinite(a) & ~z
    return bool(np.all(np.abs(a[f] - b[f]) <= rel * np.abs(b[f])))
