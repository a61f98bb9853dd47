"""Writes tests/golden/math_mpmath.json: arguments of the skeleton's own fp64
math routines and their exact results from mpmath at 40 digits.

The device accuracy test (tests/test_gpu_math.py) measures 10^6 arguments per
routine against numpy long double (a 64-bit mantissa, 2^11 times finer than
double); this fixture pins that long double reference to mpmath on 256
arguments per routine, edge cases included (tests/test_math.py), and the
device results on the same arguments directly.

    python tests/golden/make_math_fixture.py
"""
from __future__ import annotations

import json
from pathlib import Path

import mpmath as mp
import numpy as np

mp.mp.dps = 40
OUT = Path(__file__).resolve().parent / "math_mpmath.json"
TWO_PI = 6.283185307179586  # the reference's literal (Philox.java:74)


def u32_args(rng) -> list[int]:
    edges = [0, 1, 2, 2**31 - 1, 2**31, 2**32 - 3, 2**32 - 2, 2**32 - 1, 2**30, 3 * 2**30]
    sectors = [(j * 2**23 + 2**22 + o) % 2**32 for j in (0, 1, 127, 128, 255, 256, 383, 511) for o in (-1, 0, 1)]
    near_one = [2**32 - 1 - k * 997 for k in range(8)]
    rand = [int(v) for v in rng.integers(0, 2**32, 256 - len(edges) - len(sectors) - len(near_one), dtype=np.uint64)]
    return edges + sectors + near_one + rand


def s(v) -> str:
    return mp.nstr(v, 36, strip_zeros=False)


def main() -> None:
    rng = np.random.default_rng(20261202)
    c = u32_args(rng)
    u = [(mp.mpf(k) + mp.mpf(0.5)) / mp.mpf(2) ** 32 for k in c]
    theta = [float(np.float64(TWO_PI) * np.float64((k + 0.5) * 2.0**-32)) for k in c]
    x = [0.0, -0.0, 1e-300, 5e-324, 708.0, -708.0, 0.5, -0.5, 1.0, -1.0]
    x += list(rng.uniform(-0.5, 0.5, 100)) + list(rng.uniform(-30, 30, 80)) + list(rng.uniform(-708, 708, 66))
    a = [2.2250738585072014e-308, 1.0, 2.0, 0.25, 1.7976931348623157e308]
    a += list(np.exp(rng.uniform(np.log(2.3e-308), np.log(1.7e308), 251)))
    b = [2.0**-1022, 2.0**1022, 1.0, -3.0, -2.0**-1022]
    b += list(np.exp(rng.uniform(np.log(2.3e-308), np.log(4.4e307), 200))) + \
        list(-np.exp(rng.uniform(np.log(2.3e-308), np.log(4.4e307), 51)))
    out = {
        "about": "mpmath (40 digits) values of the skeleton routines' exact results; written by "
                 "tests/golden/make_math_fixture.py",
        "neg2log": {"c": c, "value": [s(-2 * mp.log(ui)) for ui in u]},
        "sincos": {"c": c, "theta": [float.hex(t) for t in theta],
                   "sin": [s(mp.sin(mp.mpf(t))) for t in theta], "cos": [s(mp.cos(mp.mpf(t))) for t in theta]},
        "exp": {"x": [float.hex(float(v)) for v in x], "value": [s(mp.exp(mp.mpf(float(v)))) for v in x]},
        "sqrt": {"a": [float.hex(float(v)) for v in a], "value": [s(mp.sqrt(mp.mpf(float(v)))) for v in a],
                 "half_rsqrt": [s(mp.mpf(0.5) / mp.sqrt(mp.mpf(float(v)))) for v in a]},
        "recip": {"b": [float.hex(float(v)) for v in b], "value": [s(mp.mpf(1) / mp.mpf(float(v))) for v in b]},
    }
    OUT.write_text(json.dumps(out, indent=0) + "\n")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
