"""The C++ host layer (recording API, engine SPI, selection) on the CPU.

Mirrors the reference's own behaviour: engines that cannot run are absent from
selection rather than failing it (AadEngines.java:41-98); a required engine
that is unusable raises with the list of usable ones; tapes an engine cannot
run are declined with UnsupportedOperationException (AadEngine.java:56-86).
"""
from __future__ import annotations

import numpy as np
import pytest

from conftest import gpu_available


def test_recorder_records_in_java_order(nt):
    def body(rec):
        x = rec.input("x", 2.0)
        y = rec.input("y", 3.0)
        z = rec.randn()
        w = x.mul(y).add(z.mul(0.5)).exp().max(1.0)
        rec.output(w)

    t = nt.AadRecorder.record(body)
    f = t.flat()
    ops = [nt.AadOpEnum(int(o)).name for o in f["op"]]
    assert ops == ["INPUT", "INPUT", "RANDN", "MUL", "CONST", "MUL", "ADD", "EXP", "CONST", "MAX"]
    assert list(f["input_node"]) == [0, 1] and list(f["output_node"]) == [9]
    assert t.inputNames() == ["x", "y"] and t.recordedInputs() == [2.0, 3.0]
    assert list(f["active"]) == [1, 1, 0, 1, 0, 0, 1, 1, 0, 1]
    assert f["constant"][4] == 0.5 and f["constant"][0] == 2.0


def test_named_streams_and_outputs_are_extended(nt):
    def body(rec):
        x = rec.input("x", 1.0)
        s = rec.stream("jumps")
        rec.output("a", x.mul(s.randn()))
        rec.output("b", x.add(rec.randu()))

    t = nt.AadRecorder.record(body)
    assert t.hasExtendedRandom() and t.randStreamCount() == 2 and t.outputCount() == 2
    with pytest.raises(Exception):
        nt.AadRecorder.record(lambda rec: rec.output("v", rec.input("x", 1.0)) or rec.output("v", rec.input("y", 1.0)))


def test_market_records_follow_declared_order(nt):
    m = nt.EquityMarket.atmOneYear()
    assert m.names() == ["spot", "strike", "vol", "rate", "maturity"]
    assert m.values() == [100.0, 100.0, 0.2, 0.03, 1.0]
    assert m.withSpot(110.0).spot() == 110.0 and m.withVol(0.3).vol() == 0.3
    with pytest.raises(ValueError):
        nt.EquityMarket.create(spot=-1.0, strike=100.0, vol=0.2, rate=0.0, maturity=1.0).validated()
    h = nt.HestonMarket.create(spot=100, strike=100, rate=0.03, v0=0.04, kappa=2, theta=0.04, xi=0.5, rho=-0.7)
    assert h.names() == ["spot", "strike", "rate", "v0", "kappa", "theta", "xi", "rho"]


def test_time_grid(nt):
    g = nt.TimeGrid.uniform(4)
    assert g.isUniform() and g.fraction(0) == 0.25 and g.cumulative(3) == 1.0
    g2 = nt.TimeGrid.of([0.1, 0.5, 1.0])
    assert not g2.isUniform() and abs(g2.fraction(1) - 0.4) < 1e-15
    # an equal-gap explicit grid records the same tape as uniform(n) (TimeGridTest.java:50-63)
    m = nt.EquityMarket.atmOneYear()
    a = nt.record(nt.Products.asianCall(), m, nt.TimeGrid.uniform(8)).flat()
    b = nt.record(nt.Products.asianCall(), m, nt.TimeGrid.of([(i + 1) / 8 for i in range(8)])).flat()
    assert np.array_equal(a["op"], b["op"]) and np.array_equal(a["constant"], b["constant"])


def test_cholesky_factor(nt):
    c = nt.CorrelatedNormals.of([[1.0, 0.5], [0.5, 1.0]])
    l = np.array(c.lower())
    assert np.allclose(l @ l.T, [[1.0, 0.5], [0.5, 1.0]], atol=1e-15)
    with pytest.raises(ValueError):
        nt.CorrelatedNormals.of([[1.0, 2.0], [2.0, 1.0]])


def test_engine_registry_has_rocm_at_priority_55(nt):
    engines = nt.AadEngines.discovered()
    assert [e.name() for e in engines] == ["rocm"]
    assert engines[0].priority() == 55
    assert nt.RocmAadEngine.maxLaunchSeconds() == 0.5


@pytest.mark.skipif(gpu_available(), reason="checks selection without a device")
def test_selection_without_a_device(nt):
    opts = nt.AadOptions.defaults()
    assert nt.AadEngines.available(opts) == []
    assert not nt.RocmAadEngine().isAvailable()
    assert nt.RocmAadEngine().describe() == "ROCm/HIP · no device"
    with pytest.raises(RuntimeError, match="not usable here"):
        nt.AadEngines.require("rocm", opts)
    with pytest.raises(RuntimeError, match="no usable AAD engine"):
        nt.AadEngines.select(opts)
    with pytest.raises(RuntimeError):
        nt.MonteCarlo.of(nt.Products.asianCall()).market(nt.EquityMarket.atmOneYear()).steps(8).on("rocm").build()


@pytest.mark.skipif(gpu_available(), reason="checks the decline path without a device")
def test_engine_takes_extended_tapes(nt):
    """The rocm engine no longer declines uniforms, named streams or several
    outputs (the reference's device engines do, AadEngine.java:56-86): without
    a device the only refusal left is the missing device."""
    t = nt.AadRecorder.record(lambda rec: rec.output(rec.input("x", 1.0).add(rec.randu())))
    with pytest.raises(RuntimeError, match="no ROCm/HIP gfx950 device"):
        nt.RocmAadEngine().compile(t, nt.AadOptions.defaults())
