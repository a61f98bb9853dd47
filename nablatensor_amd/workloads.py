"""The five benchmark workloads as recorded tapes.

C1 European call (1 exact GBM step), C2 arithmetic Asian call (252 fixings),
C3 down-and-in barrier call (252 smoothed daily monitors, barrier 80,
width 1.0), C4 Heston-Asian call (504 full-truncation Euler steps, rho -0.7),
C5 worst-of call on 16 correlated GBM assets (252 steps). C1-C3 are the
reference's own products (Products.europeanCall/asianCall,
ExoticProducts.BarrierOption); C4 and C5 have no reference product and are
recorded from its building blocks (HestonModel.step, CorrelatedNormals,
GbmPath) by HestonModel::asian and WorstOfBasket::call. The C5 correlation
and vols are the fixed inputs in data/worst_of_16.json.
"""
from __future__ import annotations

import json
from pathlib import Path

DATA = Path(__file__).resolve().parent / "data"

DESCRIPTIONS = {
    "C1": ("European call, GBM, 1 exact step, ATM 1y, value + 4 Greeks", 1_000_000, 42, "fp64"),
    "C2": ("Asian call, GBM, 252 fixings, ATM 1y, value + 5 Greeks", 2_000_000, 42, "fp64"),
    "C3": ("Down-and-in barrier call, GBM, 252 daily monitors, barrier 80, width 1.0, value + 5 Greeks",
           20_000_000, 42, "fp32"),
    "C4": ("Heston-Asian call, 504 full-truncation Euler steps, value + 8 adjoints", 10_000_000, 7, "fp64"),
    "C5": ("Worst-of call on 16 correlated GBM assets, 252 steps, value + 33 adjoints, 1e6 scenarios per launch",
           1_000_000, 42, "fp32"),
    "asian_weekdays": ("Asian call, GBM, 252 weekday fixings (TimeGrid.of, non-uniform), ATM 1y, value + 5 Greeks",
                       2_000_000, 42, "fp64"),
    "local_vol": ("Asian call, 252 fixings, ATM 1y, parametric local volatility (polynomial in log-moneyness), "
                  "value + 3 + k Greeks", 2_000_000, 42, "fp64"),
}


def worst_of_inputs() -> dict:
    return json.loads((DATA / "worst_of_16.json").read_text())


def workload_tapes(steps_c4: int = 504, steps_c5: int = 252) -> dict:
    from . import _host as nt

    m = nt.EquityMarket.atmOneYear()
    barrier = nt.ExoticProducts.barrier(nt.OptionTypeEnum.CALL, nt.ExoticProducts.BarrierEnum.DOWN_IN, 80.0, 1.0)
    heston = nt.HestonMarket.create(spot=100, strike=100, rate=0.03, v0=0.04, kappa=2.0, theta=0.04, xi=0.5, rho=-0.7)
    out = {
        "C1": nt.record(nt.Products.europeanCall(), m, nt.TimeGrid.uniform(1)),
        "C2": nt.record(nt.Products.asianCall(), m, nt.TimeGrid.uniform(252)),
        "C3": nt.record(barrier, m.withVol(0.25), nt.TimeGrid.uniform(252)),
        "C4": nt.record(nt.HestonModel.asian(nt.OptionTypeEnum.CALL, 2.0, steps_c4), heston),
    }
    fx = worst_of_inputs()
    basket = nt.WorstOfBasket.market([100.0] * 16, fx["sigma"], 0.03)
    out["C5"] = nt.record(nt.WorstOfBasket.call(fx["corr"], 100.0, 1.0, steps_c5), basket)
    return out


def weekday_fixings(n: int = 252) -> list[float]:
    """n fixing times in years on weekdays of the calendar: one day apart, three
    days after every fifth fixing (a weekend), day 1 first."""
    days, d = [], 0
    for i in range(n):
        d += 3 if (i % 5 == 0 and i > 0) else 1
        days.append(d / 365.0)
    return days


def schedule_tapes() -> dict:
    """Tapes whose step schedule is recorded up front rather than repeated
    exactly: the Asian call on TimeGrid.of 252 weekday fixings (GbmPath
    records a drift and a diffusion node per step for a non-uniform grid,
    GbmPath.java:49-66, and TimeGrid.of's fractions differ in their last bits
    even where the gaps are equal)."""
    from . import _host as nt

    grid = nt.TimeGrid.of(weekday_fixings())
    return {"asian_weekdays": nt.record(nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), grid)}



LOCAL_VOL_STEPS = 252


def local_vol_coefficients(k: int) -> list[float]:
    """theta_0 .. theta_{k-1} of the local-volatility polynomial: a 20% level,
    a skew of -0.1, a smile of 0.1 per unit log-moneyness squared, then small
    alternating higher terms 0.05 (-1)^j / j^2."""
    base = [0.2, -0.1, 0.1]
    return [base[j] if j < 3 else 0.05 * (-1) ** j / (j * j) for j in range(k)]


def local_vol_asian_tape(k: int = 24, steps: int = LOCAL_VOL_STEPS):
    """An arithmetic Asian call (252 fixings, ATM 1y) under a parametric local
    volatility: per step sigma = max(theta_0 + theta_1 x + ... + theta_{k-1}
    x^{k-1}, 0.01) in the log-moneyness x = ln(S / S0), held to [-1, 1] so the
    polynomial stays bounded (Horner's rule), then
    the log-Euler GBM step with that sigma (GbmPath.step,
    GbmPath.java:89-91, with the step's drift and diffusion formed from the
    state-dependent sigma, as GbmPath's drift/diffusion hooks allow). Inputs:
    spot, strike, rate, then the k coefficients. Every value of the step
    depends on all k coefficients, so tangent mode carries k + 2 tangents
    through a Horner chain of 2 (k - 1) nodes per step (work ~ k^2) where the
    reverse sweep's rules stay linear in k: the tape on which the lowering's
    cost model picks the reverse sweep once k is large enough."""
    from . import _host as nt

    dt = 1.0 / steps
    theta0 = local_vol_coefficients(k)

    def body(rec):
        spot = rec.input("spot", 100.0)
        strike = rec.input("strike", 100.0)
        rate = rec.input("rate", 0.03)
        theta = [rec.input(f"theta{j}", theta0[j]) for j in range(k)]
        log_s0 = spot.log()
        s = spot
        acc = spot.mul(0.0)
        for _ in range(steps):
            x = s.log().sub(log_s0).max(-1.0).min(1.0)
            sigma = theta[k - 1]
            for j in range(k - 2, -1, -1):
                sigma = sigma.mul(x).add(theta[j])
            sigma = sigma.max(0.01)
            drift = rate.sub(sigma.mul(sigma).mul(0.5)).mul(dt)
            s = s.mul(drift.add(sigma.mul(dt ** 0.5).mul(rec.randn())).exp())
            acc = acc.add(s)
        payoff = acc.mul(1.0 / steps).sub(strike).max(0.0)
        rec.output(payoff.mul(rate.neg().exp()))
    return nt.AadRecorder.record(body)
