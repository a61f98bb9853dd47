"""The host layer end to end on MI355X: MonteCarlo / Nabla / AadEngines select
and drive the rocm engine through libnt_rocm.so, like the reference's own
MvpPricingTest / ModelValidation flows do with their engines."""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module", autouse=True)
def device():
    from nablatensor_amd import rocm
    assert rocm.probe() > 0, "no gfx950 device visible to libnt_rocm.so"


def test_fastest_selects_rocm(nt):
    opts = nt.AadOptions.defaults()
    assert [e.name() for e in nt.AadEngines.available(opts)] == ["rocm"]
    assert nt.AadEngines.select(opts).name() == "rocm"
    assert "gfx950" in nt.RocmAadEngine().describe()


def test_monte_carlo_asian_matches_oracle(nt, tapes):
    mc = (nt.MonteCarlo.of(nt.Products.asianCall()).market(nt.EquityMarket.atmOneYear())
          .steps(252).greeks().fp64().fastest().build())
    assert mc.engine() == "rocm" and mc.nodes() == 1536
    v = mc.run(400_000, 42)
    ref = oracle.to_result(oracle.replay_sums(tapes["C2"], 400_000, 0, 42), 400_000)
    assert abs(v.price() - ref["price"]) <= 1e-10 * abs(ref["price"])
    assert rel_err(v.gradients(), ref["gradient"], floor=1e-300) <= 1e-10
    assert v.greek("vol") == v.gradients()[2]
    assert abs(v.standardError() - ref["stderr"]) <= 1e-8 * ref["stderr"]
    mc.close()


def test_replay_safe_chunks_combine_exactly(nt, tapes):
    mc = (nt.MonteCarlo.of(nt.Products.asianCall()).market(nt.EquityMarket.atmOneYear())
          .steps(252).greeks().fp64().on("rocm").build())
    exe = mc.executable()
    exe.setMaxChunkSeconds(2e-4)  # forces many small dispatches
    chunked = exe.replaySafe(300_000, 42)
    whole = exe.replay(300_000, 0, 42)
    assert exe.measuredPathsPerSecond() > 0
    assert rel_err(chunked.rawSums(), whole.rawSums(), floor=1e-300) <= 1e-12
    assert chunked.paths() == 300_000
    mc.close()


def test_set_input_ladder_reuses_one_kernel(nt):
    """MvpPricingTest.setInputLadderReusesOneKernel: monotone call prices along a spot ladder."""
    mc = (nt.MonteCarlo.of(nt.Products.europeanCall()).market(nt.EquityMarket.atmOneYear())
          .steps(1).greeks().fp64().on("rocm").build())
    last = -np.inf
    for spot in (80.0, 90.0, 100.0, 110.0, 120.0):
        v = mc.run(mc.market().withSpot(spot), 200_000, 20260830)
        assert v.price() >= last - 1e-6
        assert 0.0 < v.greek("spot") < 1.0 + 1e-6
        last = v.price()
    mc.close()


def test_heston_model_through_nabla(nt, tapes):
    h = nt.HestonMarket.create(spot=100, strike=100, rate=0.03, v0=0.04, kappa=2.0, theta=0.04, xi=0.5, rho=-0.7)
    model = nt.modelHeston(h, nt.HestonModel.asian(nt.OptionTypeEnum.CALL, 2.0, 504))
    pricer = model.fp64().greeks().on("rocm").build()
    v = pricer.run(h, 100_000, 7)
    ref = oracle.to_result(oracle.replay_sums(tapes["C4"], 100_000, 0, 7), 100_000)
    assert abs(v.price() - ref["price"]) <= 1e-10 * abs(ref["price"])
    assert rel_err(v.gradients(), ref["gradient"], floor=1e-300) <= 1e-10
    pricer.close()


def test_fp32_monte_carlo(nt, tapes):
    mc = (nt.MonteCarlo.of(nt.Products.asianCall()).market(nt.EquityMarket.atmOneYear())
          .steps(252).greeks().fp32().on("rocm").build())
    v = mc.run(200_000, 42)
    ref = oracle.to_result(oracle.replay_sums(tapes["C2"], 200_000, 0, 42), 200_000)
    assert abs(v.price() - ref["price"]) <= 1e-5 * abs(ref["price"])
    mc.close()


def test_extended_tapes_run_on_device(nt):
    """Named streams, uniforms and two outputs through the engine: every
    output's value, standard error and Jacobian row against the oracle."""
    from conftest import two_output_tape
    t = two_output_tape(nt)
    fp64 = nt.AadOptions.defaults().withPrecision(nt.AadOptions.PrecisionEnum.FLOAT64)  # defaults are fp32
    exe = nt.AadEngines.require("rocm", fp64).compile(t, fp64)
    r = exe.replay(100_000, 0, 42)
    assert r.outputNames() == ["spot", "max"] and r.outputCount() == 2
    ref = oracle.replay_sums(t.flat(), 100_000, 0, 42, all_outputs=True).reshape(2, -1)
    for o, name in enumerate(["spot", "max"]):
        got = oracle.to_result(np.array(r.rawSums()).reshape(2, -1)[o], 100_000)
        want = oracle.to_result(ref[o], 100_000)
        assert abs(r.valueOf(name) - want["price"]) <= 1e-10 * abs(want["price"])
        assert abs(got["price"] - want["price"]) <= 1e-10 * abs(want["price"])
        for j, inp in enumerate(r.inputNames()):
            assert abs(r.gradient(name, inp) - want["gradient"][j]) <= 1e-10 * max(1.0, abs(want["gradient"][j]))
    exe.close()


def test_replay_many_spot_ladder_shares_draws(nt):
    """A spot ladder priced in one call: each rung equals a separate replay with
    that spot (bit for bit on the raw sums), prices increase along the ladder."""
    mc = (nt.MonteCarlo.of(nt.Products.asianCall()).market(nt.EquityMarket.atmOneYear())
          .steps(252).greeks().fp64().on("rocm").build())
    exe = mc.executable()
    base = [100.0, 100.0, 0.2, 0.03, 1.0]
    sets = [[s] + base[1:] for s in (90.0, 95.0, 100.0, 105.0, 110.0)]
    many = exe.replayMany(sets, 100_000, 0, 42)
    assert len(many) == 5
    prices = [r.value() for r in many]
    assert all(b > a for a, b in zip(prices, prices[1:]))
    for s, r in zip(sets, many):
        for name, v in zip(exe.tape().inputNames(), s):
            exe.setInput(name, v)
        one = exe.replay(100_000, 0, 42)
        assert np.array_equal(np.array(r.rawSums()), np.array(one.rawSums()))
    mc.close()
