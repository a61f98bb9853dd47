"""Central bump-and-revalue with common random numbers, the reference's
cross-check of the adjoint Greeks (BumpCrossCheck.run, BumpCrossCheck.java:
33-49): for every input x_j, h_j = relative_bump x max(1, |x_j|), and the
Greek is (P(x + h_j e_j) - P(x - h_j e_j)) / (2 h_j), each price a price-only
replay over the same paths and seed. The 1 + 2 n input sets (the base market,
then +h and -h per input) can be replayed one by one, as the reference does,
or as one multi-market dispatch that shares the draws
(Executable.replay_many)."""
from __future__ import annotations

import numpy as np


def central_bump_sets(x0, relative_bump: float = 5e-3):
    """The base inputs, then +h_j and -h_j for each input j in order: shape
    (1 + 2 n, n); and the bumps h (n,)."""
    x0 = np.asarray(x0, dtype=np.float64)
    n = len(x0)
    h = relative_bump * np.maximum(1.0, np.abs(x0))
    sets = np.repeat(x0[None, :], 1 + 2 * n, axis=0)
    for j in range(n):
        sets[1 + 2 * j, j] += h[j]
        sets[2 + 2 * j, j] -= h[j]
    return sets, h


def bump_greeks(prices, h):
    """Central differences from the prices of central_bump_sets' sets."""
    p = np.asarray(prices, dtype=np.float64)
    return (p[1::2][:len(h)] - p[2::2][:len(h)]) / (2.0 * np.asarray(h))
