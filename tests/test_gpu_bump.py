"""The Asian call's adjoint Greeks against central bump-and-revalue on MI355X
(the benchmark configuration's "compared against 1 + 2 x 5 central bump
replays"): 2,000,000 scenarios, seed 42, fp64; h_j = 5e-3 max(1, |x_j|) with
common random numbers (BumpCrossCheck.java:33-49).

* Every adjoint Greek (one tangent-mode dispatch) within 5e-3 max(1, |g_j|) of
  its central bump: the bar of MvpPricingTest.adjointGreeksMatchCentralBumpForAsian
  (MvpPricingTest.java:56-71, 5e-3 on the delta), held per Greek.
* The 11 price-only replays reproduce the CPU oracle's bump Greeks
  (tests/golden/asian252_central_bumps.json, written by make_bump_fixture.py)
  within 1e-7, and the adjoint dispatch its adjoint Greeks within 1e-10
  relative: the whole comparison, not only its outcome, is the oracle's.
* The same 11 input sets priced in one multi-market dispatch (shared draws)
  give the same prices bit for bit.
"""
from __future__ import annotations

import json

import numpy as np
import pytest

from conftest import GOLDEN
from nablatensor_amd import bumps

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rocm():
    from nablatensor_amd import rocm as r
    assert r.probe() > 0, "no gfx950 device visible to libnt_rocm.so"
    return r


def test_asian_adjoint_greeks_match_central_bumps(rocm, tapes):
    gold = json.loads((GOLDEN / "asian252_central_bumps.json").read_text())
    t = tapes["C2"]
    n, seed = gold["scenarios"], gold["seed"]
    print(f"case C2 fp64 adjoint vs 11 central bumps, {n} scenarios", flush=True)
    with rocm.Executable(t, rocm.options("fp64")) as x:
        sums, _ = x.replay(n, 0, seed)
    adjoint = sums[2:] / n
    sets, h = bumps.central_bump_sets(t["recorded_inputs"], gold["relative_bump"])
    assert np.array_equal(h, gold["h"])
    with rocm.Executable(t, rocm.options("fp64", adjoints=False)) as x:
        prices = []
        for s in sets:
            x.set_inputs(s)
            p, _ = x.replay(n, 0, seed)
            prices.append(p[0] / n)
        many, _ = x.replay_many(sets, n, 0, seed)
    prices = np.array(prices)
    fd = bumps.bump_greeks(prices, h)
    print("adjoint", adjoint.tolist())
    print("bump   ", fd.tolist())
    assert np.all(np.abs(fd - adjoint) <= 5e-3 * np.maximum(1.0, np.abs(adjoint))), fd - adjoint
    assert np.allclose(fd, gold["bump_greeks"], rtol=0.0, atol=1e-7), fd - np.array(gold["bump_greeks"])
    assert np.allclose(adjoint, gold["adjoint_greeks"], rtol=1e-10, atol=0.0)
    assert abs(sums[0] / n - gold["adjoint_price"]) <= 1e-10 * gold["adjoint_price"]
    assert np.array_equal(many[:, 0] / n, prices)
