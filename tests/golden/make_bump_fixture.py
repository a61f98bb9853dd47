"""Writes asian252_central_bumps.json: the CPU oracle's central bump-and-revalue
Greeks of the Asian call (252 fixings, ATM 1y, fp64, 2,000,000 scenarios, seed
42; h_j = 5e-3 max(1, |x_j|), common random numbers; BumpCrossCheck.java:33-49)
and its adjoint Greeks, for the GPU test of the same comparison
(tests/test_gpu_bump.py). About a minute on 8 cores."""
from __future__ import annotations

import json
import sys
from pathlib import Path

HERE = Path(__file__).resolve().parent
ROOT = HERE.parents[1]
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "oracle"))


def main() -> None:
    import numpy as np

    import nablatensor_amd as nt
    import oracle
    from nablatensor_amd import bumps

    flat = nt.record(nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), nt.TimeGrid.uniform(252)).flat()
    n, seed = 2_000_000, 42
    adjoint = oracle.replay_sums(flat, n, 0, seed)
    sets, h = bumps.central_bump_sets(flat["recorded_inputs"])
    prices = [oracle.replay_sums(flat, n, 0, seed, inputs=s, adjoints=False)[0] / n for s in sets]
    out = {"workload": "Asian call, 252 fixings, ATM 1y, fp64", "scenarios": n, "seed": seed,
           "relative_bump": 5e-3, "h": list(h), "inputs": list(flat["recorded_inputs"]),
           "prices": prices, "bump_greeks": list(bumps.bump_greeks(prices, h)),
           "adjoint_price": adjoint[0] / n, "adjoint_greeks": list(np.asarray(adjoint[2:]) / n)}
    (HERE / "asian252_central_bumps.json").write_text(json.dumps(out, indent=1) + "\n")
    print(json.dumps(out))


if __name__ == "__main__":
    main()
