"""Pins of the CPU oracle (oracle/nt_oracle.c) against what fixes its answers.

* Philox2x32-10 round function: the Random123 known-answer vectors.
* Keying / Box-Muller leg mapping: the reference's formula restated
  independently here in numpy, plus moments of the draws.
* The whole chain (Philox + Box-Muller + recorded tape + reverse sweep + sums):
  the Asian-call aggregates printed in the reference's evidence pack
  (docs/validation.md:56-63, docs/compare/vs-bump-and-revalue.md:39).
* Closed forms: Black-Scholes for the 1-step European (MvpPricingTest.java:40-53).
* Invariants: knock-out + knock-in = vanilla (ExoticsTest.java:55-62), adjoint
  price = price-only price (ModelsTest.java:67-68), additivity of path ranges,
  thread-count independence.
* Brute force: central differences with common random numbers on small tapes,
  per path, for every reverse rule (tests/pins.py); the reference's barrier
  adjoint-delta bump test (ExoticsTest.java:81-94) and cash digital closed
  form (ExoticsTest.java:96-107).
* Uniforms and named streams: the keying restated in numpy, and the reference's
  own statistical checks (RandomStreamsTest.java: E[U] = 1/2, E[U^4] = 1/5,
  independent streams); several outputs: sums that follow from a scaled copy.
A planted mistake in the oracle (sign of a reverse rule, a leg swap, an input
order slip) fails at least one of these; tests/test_oracle_plants.py builds
the oracle with each reverse rule made wrong in turn and checks exactly that.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import oracle
import pins
from conftest import equity_tape, reference_values, rel_err, workload_tapes


# ---- Philox ------------------------------------------------------------------

def test_philox_random123_known_answers():
    vectors = reference_values()["philox2x32_10_kat"]["vectors"]
    assert len(vectors) == 3
    for row in vectors:
        c0, c1, key, o0, o1 = (int(x, 16) for x in row)
        assert oracle.philox(c0, c1, key) == (o0, o1)


def _philox_np(c0, c1, key):
    c0 = np.uint64(c0)
    c1 = np.uint64(c1)
    for _ in range(10):
        p = np.uint64(0xD256D193) * c0
        hi, lo = p >> np.uint64(32), p & np.uint64(0xFFFFFFFF)
        c0, c1 = hi ^ np.uint64(key) ^ c1, lo
        key = (key + 0x9E3779B9) & 0xFFFFFFFF
    return int(c0), int(c1)


@pytest.mark.parametrize("path,seed", [(0, 42), (12345, 42), (0x100000003, 0x12345678FEDCBA98), (2**40 + 5, 7)])
def test_normal_keying_and_legs(path, seed):
    """Draw k of path p: counter (lo, hi ^ (k>>1)), key 0x1BD11BDA; cos leg for even k, sin for odd k."""
    lo = (path & 0xFFFFFFFF) ^ (seed & 0xFFFFFFFF)
    hi = (path >> 32) ^ (seed >> 32)
    for k in (0, 1, 2, 7, 250, 251):
        c0, c1 = _philox_np(lo, hi ^ (k >> 1), 0x1BD11BDA)
        u1 = (c0 + 0.5) * 2.0 ** -32
        u2 = (c1 + 0.5) * 2.0 ** -32
        r = math.sqrt(-2.0 * math.log(u1))
        th = 6.283185307179586 * u2
        want = r * (math.cos(th) if k % 2 == 0 else math.sin(th))
        assert oracle.normal(path, seed, k) == pytest.approx(want, rel=1e-15, abs=1e-15)


def test_normal_moments():
    z = np.array([oracle.normal(p, 42, k) for p in range(4000) for k in range(4)])
    assert abs(z.mean()) < 0.03
    assert abs(z.var() - 1.0) < 0.04
    a = np.array([oracle.normal(p, 42, 0) for p in range(8000)])
    b = np.array([oracle.normal(p, 42, 1) for p in range(8000)])
    assert abs(np.mean(a * b)) < 0.03  # the two legs of one block are uncorrelated


# ---- tape structure ----------------------------------------------------------------

def test_node_counts_match_reference(nt):
    tapes = workload_tapes(nt)
    assert tapes["C1"].size() == 26
    counts = reference_values()["tape_node_counts"]
    assert tapes["C2"].size() == counts["asian_call_252"]
    assert tapes["C3"].size() == counts["down_in_barrier_252"]
    assert tapes["C4"].size() == 15144
    assert tapes["C2"].randCount() == 252 and tapes["C4"].randCount() == 1008
    assert tapes["C5"].inputCount() == 33 and tapes["C5"].randCount() == 16 * 252


def test_activity_matches_reference_rule(nt, tapes):
    for name in ("C1", "C2", "C3"):
        assert np.array_equal(oracle.active(tapes[name]), tapes[name]["active"])
    assert int(tapes["C2"]["active"].sum()) == 1279
    assert int(tapes["C3"]["active"].sum()) == 2792


# ---- whole chain: reference-held aggregates ------------------------------------------------

NAMES = ["spot", "strike", "vol", "rate", "maturity"]  # tape input order = EquityMarket field order


def test_published_asian_aggregates_1m(tapes):
    ref = reference_values()["asian_call_252_atm_1y_fp64_seed42"]["scenarios_1000000"]
    r = oracle.to_result(oracle.replay_sums(tapes["C2"], 1_000_000, 0, 42), 1_000_000)
    assert r["price"] == pytest.approx(ref["price"], rel=ref["rel_precision"])
    for j, name in enumerate(NAMES):
        assert r["gradient"][j] == pytest.approx(ref[name], rel=ref["rel_precision"]), name


def test_published_asian_aggregates_2m(tapes):
    ref = reference_values()["asian_call_252_atm_1y_fp64_seed42"]["scenarios_2000000"]
    r = oracle.to_result(oracle.replay_sums(tapes["C2"], 2_000_000, 0, 42), 2_000_000)
    assert r["price"] == pytest.approx(ref["price"], abs=ref["abs_precision"])
    for j, name in enumerate(NAMES):
        if name in ref:
            assert r["gradient"][j] == pytest.approx(ref[name], abs=ref["abs_precision"]), name


# ---- closed forms and invariants ---------------------------------------------------------------

def _bs_call(s, k, vol, r, t):
    d1 = (math.log(s / k) + (r + 0.5 * vol * vol) * t) / (vol * math.sqrt(t))
    d2 = d1 - vol * math.sqrt(t)
    n = lambda x: 0.5 * math.erfc(-x / math.sqrt(2.0))
    disc = math.exp(-r * t)
    pdf = math.exp(-0.5 * d1 * d1) / math.sqrt(2 * math.pi)
    return {"price": s * n(d1) - k * disc * n(d2), "delta": n(d1), "dK": -disc * n(d2),
            "vega": s * pdf * math.sqrt(t), "rho": k * t * disc * n(d2)}


def test_european_matches_black_scholes(tapes):
    n = 400_000
    r = oracle.to_result(oracle.replay_sums(tapes["C1"], n, 0, 20260830), n)
    bs = _bs_call(100.0, 100.0, 0.2, 0.03, 1.0)
    g = r["gradient"]
    # MvpPricingTest.java:47-51 tolerances
    assert abs(r["price"] - bs["price"]) < 0.15
    assert abs(g[0] - bs["delta"]) < 0.02
    assert abs(g[1] - bs["dK"]) < 0.02
    assert abs(g[2] - bs["vega"]) < 0.6
    assert abs(g[3] - bs["rho"]) < 0.6
    # and tighter: within 4 standard errors on the price
    assert abs(r["price"] - bs["price"]) < 4 * r["stderr"]


def test_european_per_path_by_hand(tapes):
    """One path of the 1-step European evaluated from the formula."""
    vals, grads = oracle.replay_paths(tapes["C1"], 3, 11, 42)
    for i in range(3):
        z = oracle.normal(11 + i, 42, 0)
        s, k, v, r, t = 100.0, 100.0, 0.2, 0.03, 1.0
        st = s * math.exp((r - 0.5 * v * v) * t + v * math.sqrt(t) * z)
        disc = math.exp(-r * t)
        assert vals[i] == pytest.approx(max(st - k, 0.0) * disc, rel=1e-13, abs=1e-13)
        if st > k:
            assert grads[i][0] == pytest.approx(st / s * disc, rel=1e-12)          # delta
            assert grads[i][1] == pytest.approx(-disc, rel=1e-12)                  # dV/dK
            assert grads[i][2] == pytest.approx(st * (-v * t + math.sqrt(t) * z) * disc, rel=1e-12)
            assert grads[i][3] == pytest.approx(st * t * disc - t * (st - k) * disc, rel=1e-12)


def test_knock_out_plus_knock_in_is_vanilla(nt):
    m = nt.EquityMarket.atmOneYear()
    B = nt.ExoticProducts.BarrierEnum
    mk = lambda kind: equity_tape(nt, nt.ExoticProducts.barrier(nt.OptionTypeEnum.CALL, kind, 130.0, 1.0), m, 32).flat()
    out = oracle.replay_sums(mk(B.UP_OUT), 50_000, 0, 42)
    inn = oracle.replay_sums(mk(B.UP_IN), 50_000, 0, 42)
    van = oracle.replay_sums(equity_tape(nt, nt.Products.europeanCall(), m, 32).flat(), 50_000, 0, 42)
    assert abs(out[0] + inn[0] - van[0]) <= 1e-9 * (1 + abs(van[0]))
    assert rel_err(out[2:] + inn[2:], van[2:], floor=1.0) <= 1e-9


def test_adjoint_price_equals_price_only(tapes):
    a = oracle.replay_sums(tapes["C4"], 2000, 0, 7, adjoints=True)
    b = oracle.replay_sums(tapes["C4"], 2000, 0, 7, adjoints=False)
    assert a[0] == b[0] and a[1] == b[1]


def test_ranges_and_threads_are_consistent(tapes):
    t = tapes["C2"]
    whole = oracle.replay_sums(t, 6000, 100, 42, threads=1)
    split = oracle.replay_sums(t, 2500, 100, 42, threads=1) + oracle.replay_sums(t, 3500, 2600, 42, threads=1)
    assert rel_err(split, whole, floor=1e-300) <= 1e-13
    many = oracle.replay_sums(t, 6000, 100, 42, threads=7)
    assert rel_err(many, whole, floor=1e-300) <= 1e-13


@pytest.mark.parametrize("name,idx,bump", [("C1", 0, 1e-3), ("C1", 2, 1e-5), ("C2s", 0, 1e-3), ("C2s", 3, 1e-5),
                                            ("C4s", 4, 1e-5), ("C4s", 7, 1e-5)])
def test_adjoint_matches_central_difference(nt, tapes, name, idx, bump):
    """Per-path adjoints vs central differences with the same draws (fp64)."""
    if name == "C2s":
        flat = equity_tape(nt, nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), 8).flat()
    elif name == "C4s":
        h = nt.HestonMarket.create(spot=100, strike=100, rate=0.03, v0=0.04, kappa=2.0, theta=0.04, xi=0.5, rho=-0.7)
        flat = nt.record(nt.HestonModel.asian(nt.OptionTypeEnum.CALL, 2.0, 6), h).flat()
    else:
        flat = tapes[name]
    x0 = np.array(flat["recorded_inputs"])
    vals, grads = oracle.replay_paths(flat, 64, 5, 42)
    h = bump * max(1.0, abs(x0[idx]))
    up, dn = x0.copy(), x0.copy()
    up[idx] += h
    dn[idx] -= h
    vu, _ = oracle.replay_paths(flat, 64, 5, 42, inputs=up)
    vd, _ = oracle.replay_paths(flat, 64, 5, 42, inputs=dn)
    fd = (vu - vd) / (2 * h)
    smooth = (np.abs(vals) > 1e-3) & (np.abs(vu - vd) < 0.5)  # away from the payoff kink
    assert smooth.sum() > 10
    assert np.max(np.abs(fd[smooth] - grads[smooth, idx]) / np.maximum(1.0, np.abs(grads[smooth, idx]))) < 1e-5


@pytest.mark.parametrize("name", list(pins.DERIVATIVE_CHECKS))
def test_derivative_pins(nt, name):
    """The oracle's adjoints against what fixes them from outside the reverse
    sweep (tests/pins.py): per-path central differences with common random
    numbers on the European, an 8-fixing Asian, a 6-step Heston-Asian, a
    16-monitor down-and-in barrier (DIV's second operand), an 8-step worst-of
    on 16 assets (MIN) and random tapes using every operation (ABS, LOG, MIN,
    MAX, DIV), each at 1e-5 relative; and the reference's barrier
    adjoint-delta test (ExoticsTest.java:81-94)."""
    ok, detail = pins.DERIVATIVE_CHECKS[name](nt)
    print(name, detail)
    assert ok, detail


def test_digital_matches_closed_form(nt):
    """ExoticsTest.cashDigitalMatchesBlackScholes (ExoticsTest.java:96-107):
    the smoothed cash digital within 0.03 of e^{-rT} N(d2)."""
    ok, detail = pins.check_digital_closed_form(nt)
    assert ok, detail


def test_fp32_mode_rounds_every_node(tapes):
    """fp32 replay stays within float rounding of the fp64 replay, per path."""
    v64, g64 = oracle.replay_paths(tapes["C2"], 256, 0, 42)
    v32, g32 = oracle.replay_paths(tapes["C2"], 256, 0, 42, f32=True)
    assert rel_err(v32, v64) < 1e-4
    assert not np.array_equal(v32, v64)
    assert np.all(v32.astype(np.float32) == v32)  # stored values are floats


# ---- uniforms and named streams -------------------------------------------------------

@pytest.mark.parametrize("stream,k", [(0, 0), (0, 5), (1, 0), (3, 7)])
def test_uniform_and_stream_keying(stream, k):
    """Uniform k of stream s: counter (lo, hi ^ s*0x9E3779B1 ^ (k | 2^30)),
    u = (c0 + 0.5) 2^-32 (Philox.java:44-52,81-94); normals of stream s use the
    same hi word."""
    path, seed = 0x100000003, 42
    lo = (path & 0xFFFFFFFF) ^ (seed & 0xFFFFFFFF)
    hi = ((path >> 32) ^ (seed >> 32)) ^ ((stream * 0x9E3779B1) & 0xFFFFFFFF)
    c0, _ = _philox_np(lo, hi ^ (k | 0x40000000), 0x1BD11BDA)
    assert oracle.uniform(path, seed, k, stream) == (c0 + 0.5) * 2.0 ** -32
    c0, c1 = _philox_np(lo, hi ^ (k >> 1), 0x1BD11BDA)
    r = math.sqrt(-2.0 * math.log((c0 + 0.5) * 2.0 ** -32))
    th = 6.283185307179586 * ((c1 + 0.5) * 2.0 ** -32)
    want = r * (math.cos(th) if k % 2 == 0 else math.sin(th))
    assert oracle.normal(path, seed, k, stream) == pytest.approx(want, rel=1e-15, abs=1e-15)


def test_uniforms_are_a_unit_interval_sample():
    """RandomStreamsTest.uniformDrawHasTheRightMeanAndRange: E[U] = 1/2,
    E[U^4] = 1/5, every draw in (0, 1)."""
    u = np.array([oracle.uniform(p, 0xC0FFEE, 0) for p in range(60_000)])
    assert abs(u.mean() - 0.5) < 5e-3 and abs(np.mean(u ** 4) - 0.2) < 5e-3
    assert u.min() > 0.0 and u.max() < 1.0


def test_named_streams_are_independent():
    """RandomStreamsTest.namedStreamsAreIndependent: E[z_a z_b] ~ 0 across
    streams; stream 0 is the default stream, and uniforms never reuse a
    normal's Philox block."""
    za = np.array([oracle.normal(p, 0xC0FFEE, 0, 1) for p in range(40_000)])
    zb = np.array([oracle.normal(p, 0xC0FFEE, 0, 2) for p in range(40_000)])
    assert abs(np.mean(za * zb)) < 2e-2
    assert not np.array_equal(za, zb)
    u0 = np.array([oracle.uniform(p, 7, 0) for p in range(2000)])
    z0 = np.array([oracle.normal(p, 7, 0) for p in range(2000)])
    assert abs(np.corrcoef(u0, z0)[0, 1]) < 0.1


def test_multi_output_sums_are_one_sweep_per_output(nt):
    """A tape whose second output is twice the first: its sums (values,
    squares x4, adjoints) follow exactly from the first output's."""
    def body(rec):
        x = rec.input("x", 1.5)
        y = x.mul(rec.randn()).exp()
        rec.output("y", y)
        rec.output("2y", y.mul(2.0))
    flat = nt.AadRecorder.record(body).flat()
    s = oracle.replay_sums(flat, 5000, 0, 3, all_outputs=True).reshape(2, -1)
    assert s[1][0] == 2 * s[0][0] and s[1][1] == 4 * s[0][1] and s[1][2] == 2 * s[0][2]
    v, g = oracle.replay_paths(flat, 50, 0, 3, output=None)
    assert np.array_equal(v[:, 1], 2 * v[:, 0]) and np.array_equal(g[:, 1, :], 2 * g[:, 0, :])


def test_path_ranges_wrap_modulo_two_to_the_64(tapes):
    """Path indices are offset + i modulo 2^64 (the reference's long
    arithmetic): a range that crosses 2^64 is the range up to it plus the
    range from 0, whichever worker thread's chunk holds the crossing."""
    t = tapes["C2"]
    for threads in (1, 16):
        whole = oracle.replay_sums(t, 4000, 2**64 - 1500, 11, threads=threads)
        head = oracle.replay_sums(t, 1500, 2**64 - 1500, 11, threads=threads)
        tail = oracle.replay_sums(t, 2500, 0, 11, threads=threads)
        assert np.allclose(whole, head + tail, rtol=1e-12, atol=0.0)


# ---- standard error: AadTotals.toResult against the per-path rows -----------------------

@pytest.mark.parametrize("name,paths", [("C1", 4000), ("C2", 3000), ("C3", 2000), ("C4", 800)])
def test_sums_and_stderr_match_the_per_path_rows(tapes, name, paths):
    """The raw sums are the sums of the per-path rows (sum y, sum y^2, sum of
    each adjoint) and the standard error of AadTotals.toResult
    (AadTotals.java:68-89), sqrt(max(0, (sum y^2 - n ybar^2) / (n - 1)) / n), is
    the sample standard deviation of the rows over sqrt(n): a wrong square, a
    missing root or n in place of n - 1 fails. Both the Python and the C
    restatement are checked."""
    t = tapes[name]
    seed = 7 if name == "C4" else 42
    sums = oracle.replay_sums(t, paths, 0, seed)
    v, g = oracle.replay_paths(t, paths, 0, seed)
    assert sums[0] == pytest.approx(v.sum(), rel=1e-12)
    assert sums[1] == pytest.approx(np.sum(v * v), rel=1e-12)
    assert np.allclose(sums[2:], g.sum(axis=0), rtol=1e-12, atol=1e-12 * np.abs(g).sum())
    want = np.std(v, ddof=1) / np.sqrt(paths)
    assert want > 0
    for res in (oracle.to_result(sums, paths), oracle.to_result_c(sums, paths, g.shape[1])):
        assert res["stderr"] == pytest.approx(want, rel=1e-10)
        assert res["price"] == pytest.approx(v.mean(), rel=1e-12)
        assert np.allclose(res["gradient"], g.mean(axis=0), rtol=1e-12, atol=1e-14)
    # one scenario has no standard error
    assert np.isnan(oracle.to_result(sums, 1)["stderr"]) and np.isnan(oracle.to_result_c(sums, 1, 0)["stderr"])


# ---- Merton jump-diffusion: uniforms against a closed form ------------------------------

MERTON = dict(spot=100.0, strike=100.0, vol=0.18, rate=0.03, maturity=1.0, jumpIntensity=0.75, jumpMean=-0.05,
              jumpVol=0.15)


def test_merton_series_reduces_to_black_scholes():
    """The Poisson series with no jumps is the Black-Scholes call: 9.4134 for
    S = K = 100, sigma 0.2, r 0.03, T 1 (d1 = 0.25, d2 = 0.05)."""
    from conftest import merton_series_call
    from math import erf, exp, log, sqrt
    ncdf = lambda x: 0.5 * (1.0 + erf(x / sqrt(2.0)))
    d1 = (log(1.0) + (0.03 + 0.02) * 1.0) / 0.2
    bs = 100.0 * ncdf(d1) - 100.0 * exp(-0.03) * ncdf(d1 - 0.2)
    assert merton_series_call(100, 100, 1.0, 0.03, 0.2, 0.0, -0.1, 0.2) == pytest.approx(bs, rel=1e-14)
    assert bs == pytest.approx(9.4134, abs=1e-4)


def test_merton_monte_carlo_converges_to_the_poisson_series(nt):
    """JumpModelsTest.mertonMonteCarloConvergesToThePoissonSeries
    (JumpModelsTest.java:46-53; docs/examples/jump-models.md:48-50): the Merton
    tape (a uniform per step decides the jump) within 1.5% of the exact
    Poisson-series price. A uniform that reused a normal's Philox block (a
    missing 2^30 tag) would tie the jump to the largest diffusion moves and
    fail it."""
    from conftest import merton_call_tape, merton_series_call
    flat = merton_call_tape(nt, MERTON).flat()
    paths = 400_000
    res = oracle.to_result(oracle.replay_sums(flat, paths, 0, 42), paths)
    exact = merton_series_call(100, 100, 1.0, 0.03, 0.18, 0.75, -0.05, 0.15)
    assert abs(res["price"] - exact) <= 0.015 * exact, (res["price"], exact)


def test_merton_without_jumps_is_black_scholes(nt):
    """JumpModelsTest.mertonCollapsesToBlackScholesWhenIntensityIsZero
    (JumpModelsTest.java:56-62): intensity 0 gives the Black-Scholes call
    within 2%."""
    from conftest import merton_call_tape, merton_series_call
    m = dict(MERTON, vol=0.2, jumpIntensity=0.0, jumpMean=-0.1, jumpVol=0.2)
    flat = merton_call_tape(nt, m, steps=64).flat()
    res = oracle.to_result(oracle.replay_sums(flat, 200_000, 0, 7), 200_000)
    bs = merton_series_call(100, 100, 1.0, 0.03, 0.2, 0.0, -0.1, 0.2)
    assert abs(res["price"] - bs) <= 0.02 * bs, (res["price"], bs)


def test_merton_adjoint_spot_delta_matches_bump(nt):
    """JumpModelsTest.mertonAdjointSpotDeltaMatchesBump (JumpModelsTest.java:
    75-87): the adjoint spot delta against a central bump of 1.0 with common
    random numbers, within 5e-3 (1 + |bump|); the jumpMean adjoint within 8%."""
    from conftest import merton_call_tape
    m = dict(MERTON, jumpIntensity=0.8)
    flat = merton_call_tape(nt, m, steps=64).flat()
    paths, seed = 100_000, 42
    base = np.array([m[f] for f in ("spot", "strike", "vol", "rate", "maturity", "jumpIntensity", "jumpMean",
                                    "jumpVol")])
    adj = oracle.to_result(oracle.replay_sums(flat, paths, 0, seed, inputs=base), paths)["gradient"]
    for j, h, tol in ((0, 1.0, 5e-3), (6, 5e-3, 0.08)):
        up, dn = base.copy(), base.copy()
        up[j] += h
        dn[j] -= h
        pu = oracle.replay_sums(flat, paths, 0, seed, inputs=up, adjoints=False)[0] / paths
        pd = oracle.replay_sums(flat, paths, 0, seed, inputs=dn, adjoints=False)[0] / paths
        bump = (pu - pd) / (2 * h)
        assert abs(adj[j] - bump) <= tol * (1 + abs(bump)), (j, adj[j], bump)
