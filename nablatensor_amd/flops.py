"""Algorithmic FLOPs per scenario of a tape under the NT-FLOP v1 convention.

The convention prices one scenario of a replay (draws + forward + reverse):
  forward   ADD SUB MUL DIV MAX MIN = 1; NEG ABS CONST INPUT = 0;
            EXP LOG = 20 (fp64) / 6 (fp32); SQRT = 8 / 3
  draws     per Philox block: 8 + LOG + SQRT + sincos (40 fp64 / 12 fp32);
            the integer Philox rounds count 0
  reverse   per active node and active operand: ADD SUB 1, MUL 2,
            DIV 2 (first operand) / 3 (second), NEG 1, EXP 2, LOG 2, SQRT 3,
            ABS 1, MAX MIN 1
Recomputation done by a checkpointed kernel is executed work, not counted.
`achieved = flops_per_scenario * scenarios / kernel_seconds` is what the
roofline fraction is measured against (78.6 TFLOP/s fp64 vector peak; fp32 is
priced against the same 157.3 TFLOP/s headline even though packed fp32 is not
used).
"""
from __future__ import annotations

import numpy as np

CONST, INPUT, RANDN, RANDU, ADD, SUB, MUL, DIV, NEG, EXP, LOG, SQRT, MAX, MIN, ABS = range(15)

PEAK_TFLOPS = {"fp64": 78.6, "fp32": 157.3}


def flops_per_scenario(flat: dict, precision: str = "fp64", adjoints: bool = True) -> int:
    op = np.asarray(flat["op"])
    a = np.asarray(flat["arg_a"])
    b = np.asarray(flat["arg_b"])
    active = np.asarray(flat["active"]).astype(bool)
    f64 = precision == "fp64"
    trans = 20 if f64 else 6
    sq = 8 if f64 else 3
    sincos = 40 if f64 else 12
    fwd = {ADD: 1, SUB: 1, MUL: 1, DIV: 1, MAX: 1, MIN: 1, EXP: trans, LOG: trans, SQRT: sq}
    total = 0
    for o, n in zip(*np.unique(op, return_counts=True)):
        total += fwd.get(int(o), 0) * int(n)
    # distinct Philox blocks (counter = ordinal >> 1) per stream
    draws = a[op == RANDN]
    blocks = len(np.unique(draws >> 1))
    total += blocks * (8 + trans + sq + sincos)
    if not adjoints:
        return total
    one = {ADD: (1, 1), SUB: (1, 1), MUL: (2, 2), DIV: (2, 3), NEG: (1, 0), EXP: (2, 0), LOG: (2, 0),
           SQRT: (3, 0), ABS: (1, 0), MAX: (1, 1), MIN: (1, 1)}
    unary = {NEG, EXP, LOG, SQRT, ABS}
    for i in np.nonzero(active)[0]:
        o = int(op[i])
        if o not in one:
            continue
        ca, cb = one[o]
        if active[a[i]]:
            total += ca
        if o not in unary and active[b[i]]:
            total += cb
    return int(total)
