"""The skeleton's own fp64 math (nt_skeleton.h) as compiled for gfx950, on the
device, over 10^6 arguments per routine plus the fixture's edge cases.

The host tests (test_math.py) run the same source with stand-ins for the
hardware seeds (v_rsq_f64, v_rcp_f64) that carry a pseudo-random relative
error of up to 2^-22; these run the real instructions. References: numpy long double (pinned to mpmath at 40 digits in
test_math.py) for the random arguments, mpmath values from
tests/golden/math_mpmath.json for the fixture's. Bounds: -2 ln u within
2 ulp, ln a of a LOG node within 2 ulp (the flag set off the positive normals), sin and cos of the reference's rounded angle within 2 * 2^-53
absolute, exp within 1 ulp for |x| <= 708 (the range flag set outside it),
sqrt within 1 ulp and 1 / (2 sqrt) within 2 ulp for positive normals, 1/b
within 1 ulp for 2^-1022 <= |b| <= 2^1022 (the flag set outside); the
Box-Muller pair within 4e-15 of the oracle's glibc draws.
"""
from __future__ import annotations

import ctypes as C
import json

import mpmath as mp
import numpy as np
import pytest

import oracle
from conftest import ROOT

pytestmark = pytest.mark.gpu

LIB = ROOT / "tests" / "device_math" / "libnt_math_device.so"
N = 1_000_000
LD = np.longdouble
mp.mp.dps = 40


@pytest.fixture(scope="module")
def dm():
    from nablatensor_amd import rocm
    assert rocm.probe() > 0, "no gfx950 device"
    assert LIB.exists(), f"{LIB} is missing: run the build"
    L = C.CDLL(str(LIB))
    P = C.POINTER
    L.dm_neg2log.argtypes = [P(C.c_uint32), P(C.c_double), C.c_long]
    L.dm_sincos.argtypes = [P(C.c_uint32), P(C.c_double), P(C.c_double), C.c_long]
    L.dm_exp.argtypes = [P(C.c_double), P(C.c_double), P(C.c_int), C.c_long]
    L.dm_log.argtypes = [P(C.c_double), P(C.c_double), P(C.c_int), C.c_long]
    L.dm_sqrt_q.argtypes = [P(C.c_double), P(C.c_double), P(C.c_double), P(C.c_int), C.c_long]
    L.dm_recip.argtypes = [P(C.c_double), P(C.c_double), P(C.c_int), C.c_long]
    L.dm_normal_pair.argtypes = [P(C.c_uint32)] * 3 + [P(C.c_double)] * 2 + [C.c_long]
    return L


@pytest.fixture(scope="module")
def fx():
    return json.loads((ROOT / "tests" / "golden" / "math_mpmath.json").read_text())


def _p(a, t):
    return a.ctypes.data_as(C.POINTER(t))


def ulps(got, ref):
    """|got - ref| in ulps of the double nearest ref (long double arithmetic)."""
    unit = np.spacing(np.abs(ref.astype(np.float64)))
    unit = np.where(unit == 0, 5e-324, unit)
    return np.asarray(np.abs(got.astype(LD) - ref) / unit.astype(LD), dtype=np.float64)


def mp_ulps(got, exact_strings, absolute=False):
    worst = 0.0
    for g, v in zip(got, exact_strings):
        e = mp.mpf(v)
        unit = mp.mpf(2.0**-53) if absolute else mp.mpf(float(np.spacing(abs(float(e)))) or 5e-324)
        worst = max(worst, float(abs(mp.mpf(float(g)) - e) / unit))
    return worst


def test_neg2log_within_two_ulp(dm, fx):
    rng = np.random.default_rng(11)
    c = np.concatenate([np.array(fx["neg2log"]["c"], dtype=np.uint64), rng.integers(0, 2**32, N, dtype=np.uint64),
                        2**32 - 1 - np.arange(0, 2_000_000, 97, dtype=np.uint64)])
    c32 = np.ascontiguousarray(c, dtype=np.uint32)
    out = np.zeros(len(c))
    print(f"case neg2log n={len(c)}", flush=True)
    assert dm.dm_neg2log(_p(c32, C.c_uint32), _p(out, C.c_double), len(c)) == 0
    u = (c.astype(np.float64) + 0.5) * 2.0**-32
    err = ulps(out, -2 * np.log(u.astype(LD)))
    k = len(fx["neg2log"]["c"])
    exact = mp_ulps(out[:k], fx["neg2log"]["value"])
    print(f"neg2log worst {err.max():.3f} ulp (fixture vs mpmath {exact:.3f})")
    assert err.max() <= 2.0 and exact <= 2.0


def test_sincos_within_two_units_of_2_pow_minus_53(dm, fx):
    rng = np.random.default_rng(12)
    c = np.concatenate([np.array(fx["sincos"]["c"], dtype=np.uint64), rng.integers(0, 2**32, N, dtype=np.uint64)])
    c32 = np.ascontiguousarray(c, dtype=np.uint32)
    s, co = np.zeros(len(c)), np.zeros(len(c))
    print(f"case sincos n={len(c)}", flush=True)
    assert dm.dm_sincos(_p(c32, C.c_uint32), _p(s, C.c_double), _p(co, C.c_double), len(c)) == 0
    theta = np.float64(6.283185307179586) * ((c.astype(np.float64) + 0.5) * 2.0**-32)  # the reference's rounded angle
    es = np.asarray(np.abs(s.astype(LD) - np.sin(theta.astype(LD))) / LD(2.0**-53), dtype=np.float64)
    ec = np.asarray(np.abs(co.astype(LD) - np.cos(theta.astype(LD))) / LD(2.0**-53), dtype=np.float64)
    k = len(fx["sincos"]["c"])
    exact = max(mp_ulps(s[:k], fx["sincos"]["sin"], True), mp_ulps(co[:k], fx["sincos"]["cos"], True))
    print(f"sin worst {es.max():.3f}, cos worst {ec.max():.3f} x 2^-53 (fixture vs mpmath {exact:.3f})")
    assert es.max() <= 2.0 and ec.max() <= 2.0 and exact <= 2.0


def test_exp_within_one_ulp_and_its_range_flag(dm, fx):
    rng = np.random.default_rng(13)
    fixture = np.array([float.fromhex(v) for v in fx["exp"]["x"]])
    x = np.ascontiguousarray(np.concatenate([fixture, rng.uniform(-0.5, 0.5, N // 2), rng.uniform(-708, 708, N // 2),
                                             [708.0000000000001, -708.0000000000001, 709.7, -745.0, np.inf, -np.inf,
                                              np.nan]]))
    out = np.zeros(len(x))
    bad = np.zeros(len(x), dtype=np.int32)
    print(f"case exp n={len(x)}", flush=True)
    assert dm.dm_exp(_p(x, C.c_double), _p(out, C.c_double), _p(bad, C.c_int), len(x)) == 0
    with np.errstate(invalid="ignore"):
        inside = np.abs(x) <= 708.0
    assert (bad[inside] == 0).all() and (bad[~inside] == 1).all()
    err = ulps(out[inside], np.exp(x[inside].astype(LD)))
    exact = mp_ulps(out[:len(fixture)], fx["exp"]["value"])
    print(f"exp worst {err.max():.3f} ulp (fixture vs mpmath {exact:.3f})")
    assert err.max() <= 1.0 and exact <= 1.0


def test_log_within_two_ulp_and_its_range_flag(dm):
    """ln(a) of a LOG node (nt_log_fast) on the device: within 2 ulp over the
    positive normal range (10^6 arguments against long double, 300 of them
    against mpmath); zero, subnormal, negative, infinite and NaN arguments
    raise the flag."""
    rng = np.random.default_rng(17)
    x = np.ascontiguousarray(np.concatenate([
        np.exp(rng.uniform(-700.0, 700.0, N // 2)), 1.0 + rng.uniform(-2.0 ** -8, 2.0 ** -8, N // 4),
        rng.uniform(0.5, 2.0, N // 4), [2.2250738585072014e-308, 1.7976931348623157e308, 1.0],
        [0.0, -0.0, 5e-324, -1.0, np.inf, -np.inf, np.nan]]))
    special = 7
    out = np.zeros(len(x))
    bad = np.zeros(len(x), dtype=np.int32)
    print(f"case log n={len(x)}", flush=True)
    assert dm.dm_log(_p(x, C.c_double), _p(out, C.c_double), _p(bad, C.c_int), len(x)) == 0
    assert (bad[:-special] == 0).all() and (bad[-special:] == 1).all()
    xs, os_ = x[:-special], out[:-special]
    keep = xs != 1.0
    err = ulps(os_[keep], np.log(xs[keep].astype(LD)))
    assert os_[~keep].max() == 0.0
    pick = rng.choice(np.nonzero(keep)[0], 300, replace=False)
    exact = 0.0
    for i in pick:
        want = mp.log(mp.mpf(float(xs[i])))
        exact = max(exact, float(abs(mp.mpf(float(os_[i])) - want) / mp.mpf(float(np.spacing(abs(float(want)))))))
    print(f"log worst {err.max():.3f} ulp (sample vs mpmath {exact:.3f})")
    assert err.max() <= 2.0 and exact <= 2.0


def test_sqrt_and_its_tangent_factor(dm, fx):
    rng = np.random.default_rng(14)
    fixture = np.array([float.fromhex(v) for v in fx["sqrt"]["a"]])
    normals = np.concatenate([fixture, np.exp(rng.uniform(np.log(2.3e-308), np.log(1.7e308), N // 2)),
                              np.exp(rng.uniform(np.log(1e-6), np.log(10.0), N // 2))])
    special = np.array([0.0, -0.0, 5e-324, 1e-310, -1.0, -1e-300, np.inf, -np.inf, np.nan])
    a = np.ascontiguousarray(np.concatenate([normals, special]))
    out, q = np.zeros(len(a)), np.zeros(len(a))
    bad = np.zeros(len(a), dtype=np.int32)
    print(f"case sqrt_q n={len(a)}", flush=True)
    assert dm.dm_sqrt_q(_p(a, C.c_double), _p(out, C.c_double), _p(q, C.c_double), _p(bad, C.c_int), len(a)) == 0
    n = len(normals)
    assert (bad[:n] == 0).all() and (bad[n:n + 2] == 0).all() and (bad[n + 2:] == 1).all()
    es = ulps(out[:n], np.sqrt(normals.astype(LD)))
    eq = ulps(q[:n], LD(0.5) / np.sqrt(normals.astype(LD)))
    k = len(fixture)
    exact = max(mp_ulps(out[:k], fx["sqrt"]["value"]), mp_ulps(q[:k], fx["sqrt"]["half_rsqrt"]) / 2.0)
    print(f"sqrt worst {es.max():.3f} ulp, 1/(2 sqrt) worst {eq.max():.3f} ulp")
    assert es.max() <= 1.0 and eq.max() <= 2.0 and exact <= 1.0
    assert (out[n:n + 2] == 0.0).all() and np.array_equal(np.signbit(out[n:n + 2]), [False, True])
    assert np.isfinite(q[n:n + 2]).all() and (q[n:n + 2] > 1e150).all()


def test_recip_within_one_ulp_and_its_range_flag(dm, fx):
    rng = np.random.default_rng(15)
    fixture = np.array([float.fromhex(v) for v in fx["recip"]["b"]])
    mags = np.exp(rng.uniform(np.log(2.3e-308), np.log(4.4e307), N // 2))
    b = np.ascontiguousarray(np.concatenate([fixture, mags, -mags, [0.0, -0.0, 1e-310, 2.0**1023, -1.7e308, np.inf,
                                                                    -np.inf, np.nan]]))
    out = np.zeros(len(b))
    bad = np.zeros(len(b), dtype=np.int32)
    print(f"case recip n={len(b)}", flush=True)
    assert dm.dm_recip(_p(b, C.c_double), _p(out, C.c_double), _p(bad, C.c_int), len(b)) == 0
    with np.errstate(invalid="ignore"):
        ok = (np.abs(b) >= 2.0**-1022) & (np.abs(b) <= 2.0**1022)
    assert (bad[ok] == 0).all() and (bad[~ok] == 1).all()
    err = ulps(out[ok], LD(1) / b[ok].astype(LD))
    exact = mp_ulps(out[:len(fixture)], fx["recip"]["value"])
    print(f"recip worst {err.max():.3f} ulp (fixture vs mpmath {exact:.3f})")
    assert err.max() <= 1.0 and exact <= 1.0


def test_normal_pairs_track_the_oracle(dm):
    """Draws 0 and 1 of 20,000 paths from the device pair against the oracle's
    glibc evaluation of the reference formula (Philox.java:55-78)."""
    paths = np.arange(0, 20_000, dtype=np.uint64) * np.uint64(7919) + np.uint64(0x100000003)
    seed = 42
    lo = np.ascontiguousarray((paths & np.uint64(0xFFFFFFFF)) ^ np.uint64(seed), dtype=np.uint32)
    hi = np.ascontiguousarray(paths >> np.uint64(32), dtype=np.uint32)
    ctr = np.zeros(len(paths), dtype=np.uint32)
    zc, zs = np.zeros(len(paths)), np.zeros(len(paths))
    print("case normal pairs n=20000", flush=True)
    assert dm.dm_normal_pair(_p(lo, C.c_uint32), _p(hi, C.c_uint32), _p(ctr, C.c_uint32), _p(zc, C.c_double),
                             _p(zs, C.c_double), len(paths)) == 0
    ref_c = np.array([oracle.normal(int(p), seed, 0) for p in paths])
    ref_s = np.array([oracle.normal(int(p), seed, 1) for p in paths])
    print(f"pair worst {max(np.abs(zc - ref_c).max(), np.abs(zs - ref_s).max()):.2e}")
    assert np.abs(zc - ref_c).max() <= 4e-15 and np.abs(zs - ref_s).max() <= 4e-15
