"""Accuracy of the skeleton's own fp64 log / sqrt / sincos / exp
(nt_skeleton.h), built for the host, against mpmath at 40 digits; and of the
Box-Muller pair against the oracle's glibc evaluation of the reference
formula."""
from __future__ import annotations

import ctypes as C
import os
import subprocess
import tempfile
from pathlib import Path

import mpmath as mp
import numpy as np
import pytest

import oracle
from conftest import ROOT

mp.mp.dps = 40
EMU = ROOT / "tests" / "host_emu"


@pytest.fixture(scope="module")
def lib():
    out = Path(tempfile.gettempdir()) / f"nt_math_emu_{os.getpid()}.so"  # one per test worker
    subprocess.run(["g++", "-O2", "-std=c++17", "-shared", "-fPIC", "-ffp-contract=off", "-w",
                    f"-I{ROOT / 'nablatensor_amd' / 'csrc'}", f"-I{EMU}", str(EMU / "math_main.cpp"),
                    "-o", str(out)], check=True)
    L = C.CDLL(str(out))
    P = C.POINTER
    L.emu_neg2log.argtypes = [P(C.c_uint32), P(C.c_double), C.c_long]
    L.emu_log.argtypes = [P(C.c_double), P(C.c_double), P(C.c_int), C.c_long]
    L.emu_sincos.argtypes = [P(C.c_uint32), P(C.c_double), P(C.c_double), C.c_long]
    L.emu_sqrt.argtypes = [P(C.c_double), P(C.c_double), C.c_long]
    L.emu_exp.argtypes = [P(C.c_double), P(C.c_double), C.c_long]
    L.emu_sqrt_q.argtypes = [P(C.c_double), P(C.c_double), P(C.c_double), P(C.c_int), C.c_long]
    L.emu_recip.argtypes = [P(C.c_double), P(C.c_double), P(C.c_int), C.c_long]
    L.emu_normal_pair.argtypes = [P(C.c_uint32)] * 3 + [P(C.c_double)] * 2 + [C.c_long]
    return L


def _u32(a):
    return np.ascontiguousarray(a, dtype=np.uint32)


def _ptr(a, t):
    return a.ctypes.data_as(C.POINTER(t))


def ulp_err(got: float, want) -> float:
    w = float(want)
    if w == 0.0:
        return abs(got) / 5e-324
    return float(abs(mp.mpf(got) - want) / mp.mpf(np.spacing(abs(w))))


def sample_u32(n: int, seed: int) -> np.ndarray:
    rng = np.random.default_rng(seed)
    edges = [0, 1, 2, 3, 2**29 - 1, 2**29, 2**29 + 1, 2**30 - 1, 2**30, 2**31 - 1, 2**31, 3 * 2**30 - 1,
             3 * 2**30, 2**32 - 2**29 - 1, 2**32 - 2**29, 2**32 - 3, 2**32 - 2, 2**32 - 1]
    # both sides of the sine/cosine table's sector boundaries (j 2^23 +- 2^22)
    sectors = [j * 2**23 + 2**22 + o for j in range(0, 512, 17) for o in (-1, 0, 1)]
    sectors = [v % 2**32 for v in sectors]
    return _u32(np.concatenate([edges, sectors, rng.integers(0, 2**32, n, dtype=np.uint64)]))


def test_neg2log_within_two_ulp(lib):
    c = sample_u32(3000, 1)
    near_one = _u32(2**32 - 1 - np.arange(0, 200000, 997))
    c = _u32(np.concatenate([c, near_one]))
    out = np.zeros(len(c))
    lib.emu_neg2log(_ptr(c, C.c_uint32), _ptr(out, C.c_double), len(c))
    worst = 0.0
    for ci, oi in zip(c, out):
        u = (mp.mpf(int(ci)) + mp.mpf(0.5)) / mp.mpf(2) ** 32
        worst = max(worst, ulp_err(oi, -2 * mp.log(u)))
    assert worst <= 2.0, worst


def log_arguments(n: int, seed: int) -> np.ndarray:
    """Positive normal doubles over the whole exponent range, around 1 (where
    ln a is small and F = 1), at the table's sector edges and the largest and
    smallest normal numbers."""
    rng = np.random.default_rng(seed)
    a = np.concatenate([
        np.exp(rng.uniform(-700.0, 700.0, n)),
        1.0 + rng.uniform(-2.0 ** -8, 2.0 ** -8, n // 4),
        rng.uniform(0.5, 2.0, n // 4),
        np.ldexp(1.0 + np.arange(0, 257) / 256.0, rng.integers(-1000, 1000, 257)),
        [1.0, np.nextafter(1.0, 2.0), np.nextafter(1.0, 0.0), 2.0, 0.5, np.sqrt(0.5), np.sqrt(2.0),
         2.2250738585072014e-308, 1.7976931348623157e308, 1e-300, 1e300]])
    return np.ascontiguousarray(a)


def test_log_within_two_ulp_and_its_range_flag(lib):
    """ln(a) of a LOG node (nt_log_fast: -1/2 of the Box-Muller routine's
    -2 ln on a's own exponent and mantissa) within 2 ulp of mpmath over the
    positive normal range; every other argument raises the flag."""
    a = log_arguments(4000, 11)
    out = np.zeros(len(a))
    bad = np.zeros(len(a), dtype=np.int32)
    lib.emu_log(_ptr(a, C.c_double), _ptr(out, C.c_double), _ptr(bad, C.c_int), len(a))
    assert not bad.any()
    worst = max(ulp_err(o, mp.log(mp.mpf(float(x)))) for x, o in zip(a, out) if x != 1.0)
    assert worst <= 2.0, worst
    assert out[np.nonzero(a == 1.0)[0][0]] == 0.0
    sp = np.ascontiguousarray([0.0, -0.0, 5e-324, 2.2250738585072009e-308, -1.0, np.inf, -np.inf, np.nan])
    out = np.zeros(len(sp))
    bad = np.zeros(len(sp), dtype=np.int32)
    lib.emu_log(_ptr(sp, C.c_double), _ptr(out, C.c_double), _ptr(bad, C.c_int), len(sp))
    assert bad.all()


def test_sincos_within_two_ulp(lib):
    c = sample_u32(3000, 2)
    s = np.zeros(len(c))
    co = np.zeros(len(c))
    lib.emu_sincos(_ptr(c, C.c_uint32), _ptr(s, C.c_double), _ptr(co, C.c_double), len(c))
    worst = 0.0
    for ci, si, cj in zip(c, s, co):
        u = (int(ci) + 0.5) * 2.0**-32
        th = mp.mpf(6.283185307179586 * u)  # the reference's rounded angle
        # error relative to the unit circle scale: sin near 0 is judged in absolute terms
        worst = max(worst, float(abs(mp.mpf(si) - mp.sin(th)) / mp.mpf(2.0**-53)),
                    float(abs(mp.mpf(cj) - mp.cos(th)) / mp.mpf(2.0**-53)))
    assert worst <= 2.0, worst


def test_sqrt_within_one_ulp(lib):
    rng = np.random.default_rng(3)
    a = np.ascontiguousarray(np.concatenate([np.exp(rng.uniform(np.log(2e-10), np.log(46.0), 20000)),
                                             [2.3283064365386963e-10, 45.75, 1.0, 2.0, 0.5]]))
    out = np.zeros(len(a))
    lib.emu_sqrt(_ptr(a, C.c_double), _ptr(out, C.c_double), len(a))
    err = np.abs(out - np.sqrt(a)) / np.spacing(np.sqrt(a))
    assert err.max() <= 1.0


def test_sqrt_with_tangent_factor(lib):
    """nt_sqrt_q: sqrt within 1 ulp and 1/(2 sqrt) within 2 ulp for
    positive normals; +-0 give +-0 and a finite factor; every other class
    (subnormal, negative, infinite, NaN) raises the flag."""
    rng = np.random.default_rng(4)
    normals = np.exp(rng.uniform(np.log(2.3e-308), np.log(1.7e308), 20000))
    a = np.ascontiguousarray(np.concatenate([normals, [2.2250738585072014e-308, 1.0, 4.0, 0.25, 1.7976931348623157e308,
                                                       0.0, -0.0, 5e-324, 1e-310, -1.0, -1e-300, np.inf, -np.inf,
                                                       np.nan]]))
    n = len(a)
    out, q = np.zeros(n), np.zeros(n)
    bad = np.zeros(n, dtype=np.int32)
    lib.emu_sqrt_q(_ptr(a, C.c_double), _ptr(out, C.c_double), _ptr(q, C.c_double), _ptr(bad, C.c_int), n)
    ok = (a > 0) & np.isfinite(a) & (a >= 2.2250738585072014e-308)
    zero = a == 0.0
    assert (bad[ok | zero] == 0).all() and (bad[~(ok | zero)] == 1).all()
    r = np.sqrt(a[ok])
    assert (np.abs(out[ok] - r) / np.spacing(r)).max() <= 1.0
    hq = 0.5 / r
    assert (np.abs(q[ok] - hq) / np.spacing(hq)).max() <= 2.0
    assert (out[zero] == 0.0).all() and np.array_equal(np.signbit(out[zero]), np.signbit(a[zero]))
    assert np.isfinite(q[zero]).all() and (q[zero] > 1e150).all()


def test_recip_within_one_ulp_and_its_range(lib):
    """nt_recip: 1/b within 1 ulp for 2^-1022 <= |b| <= 2^1022, either sign;
    zero, subnormal, larger, infinite and NaN arguments raise the flag."""
    rng = np.random.default_rng(5)
    mags = np.exp(rng.uniform(np.log(2.3e-308), np.log(4.4e307), 20000))
    b = np.ascontiguousarray(np.concatenate([mags, -mags[:5000], [2.0**-1022, 2.0**1022, 1.0, -3.0, 0.0, -0.0, 1e-310,
                                                                  2.0**1023, -1.7e308, np.inf, -np.inf, np.nan]]))
    n = len(b)
    out = np.zeros(n)
    bad = np.zeros(n, dtype=np.int32)
    lib.emu_recip(_ptr(b, C.c_double), _ptr(out, C.c_double), _ptr(bad, C.c_int), n)
    with np.errstate(invalid="ignore"):
        ok = (np.abs(b) >= 2.0**-1022) & (np.abs(b) <= 2.0**1022)
    assert (bad[ok] == 0).all() and (bad[~ok] == 1).all()
    r = 1.0 / b[ok]
    assert (np.abs(out[ok] - r) / np.spacing(np.abs(r))).max() <= 1.0


def test_normal_pairs_track_the_reference_formula(lib):
    """The pair equals the oracle's draws (glibc log/sqrt/sin/cos of the
    rounded 2 pi u2) to within 4e-15 absolute, for draws 0 and 1 of many paths."""
    paths = np.arange(0, 4000, dtype=np.uint64) * 7919 + 0x100000003
    seed = 42
    lo = _u32((paths & 0xFFFFFFFF) ^ (seed & 0xFFFFFFFF))
    hi = _u32((paths >> 32) ^ (seed >> 32))
    ctr = _u32(np.zeros(len(paths)))
    zc = np.zeros(len(paths))
    zs = np.zeros(len(paths))
    lib.emu_normal_pair(_ptr(lo, C.c_uint32), _ptr(hi, C.c_uint32), _ptr(ctr, C.c_uint32),
                        _ptr(zc, C.c_double), _ptr(zs, C.c_double), len(paths))
    ref_c = np.array([oracle.normal(int(p), seed, 0) for p in paths])
    ref_s = np.array([oracle.normal(int(p), seed, 1) for p in paths])
    assert np.max(np.abs(zc - ref_c)) <= 4e-15
    assert np.max(np.abs(zs - ref_s)) <= 4e-15


def test_exp_within_one_ulp_and_special_values(lib):
    rng = np.random.default_rng(4)
    x = np.concatenate([rng.uniform(-0.5, 0.5, 4000), rng.uniform(-30.0, 30.0, 2000),
                        rng.uniform(-708.0, 708.0, 1000), np.arange(-64, 65) * np.log(2.0) / 64,
                        [0.0, -0.0, 1e-300, -1e-300, 5e-324, 708.0, -708.0]])
    x = np.ascontiguousarray(x)
    out = np.zeros(len(x))
    lib.emu_exp(_ptr(x, C.c_double), _ptr(out, C.c_double), len(x))
    worst = max(ulp_err(o, mp.exp(mp.mpf(float(xi)))) for xi, o in zip(x, out))
    assert worst <= 1.0, worst
    # beyond +-708, the infinities and NaN go to libm: overflow, underflow to
    # subnormals and zero, NaN propagation
    sp = np.ascontiguousarray([709.5, 710.0, 1e10, np.inf, -720.0, -745.0, -746.0, -1e10, -np.inf, np.nan])
    out = np.zeros(len(sp))
    lib.emu_exp(_ptr(sp, C.c_double), _ptr(out, C.c_double), len(sp))
    with np.errstate(over="ignore"):
        want = np.exp(sp[:-1])
    assert np.array_equal(out[:-1], want) and np.isnan(out[-1])


# ---- the long double reference of the device accuracy test ------------------------------

def long_double_refs(fx):
    """numpy long double (64-bit mantissa) values of each routine's exact result
    on the fixture's arguments, as tests/test_gpu_math.py computes them for 10^6."""
    ld = np.longdouble
    c = np.array(fx["neg2log"]["c"], dtype=np.uint64)
    u = (c.astype(np.float64) + 0.5) * 2.0**-32
    theta = np.array([float.fromhex(t) for t in fx["sincos"]["theta"]])
    x = np.array([float.fromhex(v) for v in fx["exp"]["x"]])
    a = np.array([float.fromhex(v) for v in fx["sqrt"]["a"]])
    b = np.array([float.fromhex(v) for v in fx["recip"]["b"]])
    return {"neg2log": -2 * np.log(u.astype(ld)), "sin": np.sin(theta.astype(ld)), "cos": np.cos(theta.astype(ld)),
            "exp": np.exp(x.astype(ld)), "sqrt": np.sqrt(a.astype(ld)), "half_rsqrt": ld(0.5) / np.sqrt(a.astype(ld)),
            "recip": ld(1) / b.astype(ld)}


def test_long_double_reference_is_within_a_thousandth_of_a_double_ulp():
    """The device accuracy test measures ulp errors of double results against
    numpy long double; on the fixture's arguments (tests/golden/math_mpmath.json,
    mpmath at 40 digits, edge cases included) that reference is within 1e-3 of
    a double ulp of the exact result, so it resolves errors of 1 ulp to 0.1 %."""
    import json
    fx = json.loads((ROOT / "tests" / "golden" / "math_mpmath.json").read_text())
    refs = long_double_refs(fx)
    exact = {"neg2log": fx["neg2log"]["value"], "sin": fx["sincos"]["sin"], "cos": fx["sincos"]["cos"],
             "exp": fx["exp"]["value"], "sqrt": fx["sqrt"]["value"], "half_rsqrt": fx["sqrt"]["half_rsqrt"],
             "recip": fx["recip"]["value"]}
    for name, values in exact.items():
        worst = 0.0
        for r, v in zip(refs[name], values):
            e = mp.mpf(v)
            unit = mp.mpf(2.0**-53) if name in ("sin", "cos") else mp.mpf(float(np.spacing(abs(float(e))) or 5e-324))
            worst = max(worst, float(abs(mp.mpf(str(r)) - e) / unit))
        assert worst <= 1e-3, (name, worst)
