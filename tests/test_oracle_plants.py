"""Each reverse rule of the oracle is pinned: a build with that rule made
wrong (NTO_PLANT in oracle/nt_oracle.c) is rejected by at least one of the
derivative checks of tests/pins.py, which compare the oracle's adjoints with
central differences of its own forward values and with the reference's
barrier adjoint-delta test (ExoticsTest.java:81-94). The planted builds go to
a temporary directory; the default build the other tests load has no plant.
"""
from __future__ import annotations

import pytest

import oracle
import pins

RULES = {1: "ADD b", 2: "SUB b", 3: "MUL a", 4: "DIV a", 5: "DIV b", 6: "NEG", 7: "EXP", 8: "LOG", 9: "SQRT",
         10: "ABS", 11: "MAX", 12: "MIN"}


@pytest.fixture(scope="module")
def planted(tmp_path_factory):
    out = tmp_path_factory.mktemp("planted")
    return {k: oracle.build_planted(k, out / f"libnt_oracle_plant{k}.so") for k in RULES}


@pytest.mark.parametrize("plant", sorted(RULES))
def test_every_planted_reverse_rule_is_rejected(nt, planted, plant):
    with oracle.library(planted[plant]):
        for name, check in pins.DERIVATIVE_CHECKS.items():
            ok, detail = check(nt)
            if not ok:
                print(f"plant {plant} ({RULES[plant]}) rejected by {name}: {detail}")
                return
    pytest.fail(f"no check rejects a wrong {RULES[plant]} rule")


@pytest.mark.parametrize("plant,check", [
    (5, "barrier_delta_vs_bump"),   # the reference's own test catches DIV's second operand
    (5, "down_in_barrier"),
    (12, "worst_of"),               # MIN: the adjoint reaches the wrong asset
    (12, "random_tapes"),
    (10, "random_tapes"),           # ABS
    (11, "european"),               # MAX: the payoff's floor
])
def test_named_rules_are_rejected_by_their_checks(nt, planted, plant, check):
    with oracle.library(planted[plant]):
        ok, detail = pins.DERIVATIVE_CHECKS[check](nt)
    assert not ok, (plant, check, detail)
