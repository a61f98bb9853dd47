"""Writes worst_of_16.json: the fixed inputs of the 16-asset worst-of workload.

Correlation: symmetric, off-diagonals uniform in [0.2, 0.6] from numpy's
PCG64 seeded with 42, made positive definite by flooring its eigenvalues at
1e-3 and rescaling to a unit diagonal. Vols: uniform in [0.15, 0.40] from the
same generator. The Cholesky factor is included for reference; the host layer
recomputes it (CorrelatedNormals.of) from `corr`.
Run: python nablatensor_amd/data/make_worst_of_16.py
"""
import json
from pathlib import Path

import numpy as np


def make(n: int = 16, seed: int = 42) -> dict:
    rng = np.random.default_rng(seed)
    c = np.eye(n)
    iu = np.triu_indices(n, 1)
    c[iu] = rng.uniform(0.2, 0.6, size=len(iu[0]))
    c = np.triu(c) + np.triu(c, 1).T
    w, v = np.linalg.eigh(c)
    c = (v * np.maximum(w, 1e-3)) @ v.T
    d = np.sqrt(np.diag(c))
    c = c / np.outer(d, d)
    c = 0.5 * (c + c.T)
    np.fill_diagonal(c, 1.0)
    sigma = rng.uniform(0.15, 0.40, size=n)
    lower = np.linalg.cholesky(c)
    return {"n": n, "seed": seed, "corr": c.tolist(), "sigma": sigma.tolist(), "cholesky": lower.tolist(),
            "min_eigenvalue": float(np.linalg.eigvalsh(c).min())}


if __name__ == "__main__":
    out = Path(__file__).resolve().parent / "worst_of_16.json"
    out.write_text(json.dumps(make(), indent=1))
    print("wrote", out)
