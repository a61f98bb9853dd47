"""CPU tests of the tape lowering (nablatensor_amd/csrc/lower.cpp).

The generated kernel source is compiled for the host (tests/host_emu) with the
same IEEE arithmetic as the oracle (no FMA contraction, glibc libm) and run
over an emulated grid with the device's scratch indexing. Reverse-mode fp64
results must then equal the oracle bit for bit: any slip in loop detection,
carry handling, segment checkpoints, stored values, draw pairing or the order
of adjoint accumulation shows up as a difference. Tangent mode computes the
same values bit for bit (except where a multiplicative carry, or a running
sum of one, is carried as its product of factors G: such values are held to
the per-path bar) and the same derivatives in another order, so its
gradients are held to the per-path bar instead.
"""
from __future__ import annotations

import re

import numpy as np
import pytest

import emu
import oracle
from conftest import (ABOVE, STRICT, check_per_path, degenerate_tapes, equity_tape, no_input_tape, rel_err, scaled_exp_tape,
                      sqrt_classes_tape, tape_slots)

OFFSET = 0x100000003


def carries_g_alone(src: str) -> bool:
    """The kernel carries a multiplicative carry as G alone and rebuilds its
    value as c0 G after the loop (or a running sum of it as A0 + c0 sum G):
    that value then differs from the oracle's step-by-step product by
    rounding (about sqrt(steps) ulps), and the path values are held to the
    per-path bar instead of bit equality."""
    return re.search(r"st\d+ = (v\d+ \+ )?c0_\d+ \* (gs|st)\d+;", src) is not None


def assert_values_match(v, ov, src):
    if carries_g_alone(src):
        assert rel_err(v, ov) <= 1e-12
    else:
        assert np.array_equal(v, ov)


def run_emulated(flat, opts, paths, offset=OFFSET, seed=42, grid=3, block=64, inputs=None, rocm=None):
    src = rocm.lower(flat, opts)
    k = emu.EmulatedKernel(src, len(flat["input_node"]), tape_slots(src))
    x = flat["recorded_inputs"] if inputs is None else inputs
    return k.run(x, paths, offset, seed, grid=grid, block=block)


@pytest.fixture(scope="module")
def rocm():
    from nablatensor_amd import rocm as r
    return r


@pytest.mark.parametrize("ckpt", [1, 2, 3])
@pytest.mark.parametrize("name,paths", [("C1", 700), ("C2", 400), ("C3", 300), ("C4", 150), ("C5", 40)])
def test_emulated_fp64_is_bit_exact(rocm, tapes, name, paths, ckpt):
    """With libm Box-Muller (NT_DEVICE_LIBM, glibc on the host) every fp64 bit matches."""
    flat = tapes[name]
    sums, v, g = run_emulated(flat, rocm.options("fp64", checkpoint=ckpt, libm=1, mode=1), paths, rocm=rocm)
    ov, og = oracle.replay_paths(flat, paths, OFFSET, 42, threads=1)
    assert np.array_equal(v, ov)
    assert np.array_equal(g, og)
    ref = oracle.replay_sums(flat, paths, OFFSET, 42, threads=1)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-13


@pytest.mark.parametrize("name,paths", [("C1", 700), ("C2", 400), ("C3", 300), ("C4", 150), ("C5", 40)])
def test_emulated_tangent_values_bit_exact_gradients_within_bar(rocm, tapes, name, paths):
    """Tangent mode: same forward arithmetic (values bit for bit with libm
    Box-Muller, but for a carry kept as G alone); derivatives within the
    per-path bar."""
    flat = tapes[name]
    opts = rocm.options("fp64", libm=1, mode=2)
    sums, v, g = run_emulated(flat, opts, paths, rocm=rocm)
    ov, _ = oracle.replay_paths(flat, paths, OFFSET, 42, threads=1)
    assert_values_match(v, ov, rocm.lower(flat, opts))
    check_per_path(v, g, flat, paths, OFFSET, 42, min_strict=STRICT[name], max_above=ABOVE[name])
    ref = oracle.replay_sums(flat, paths, OFFSET, 42, threads=1)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-12


@pytest.mark.parametrize("seg", [2, 4, 10, 50])
def test_segment_lengths_with_tail(rocm, tapes, seg):
    """Segment lengths that do not divide 252 leave a tail segment."""
    flat = tapes["C2"]
    _, v, g = run_emulated(flat, rocm.options("fp64", checkpoint=1, seg_len=seg, libm=1, mode=1), 200, rocm=rocm)
    ov, og = oracle.replay_paths(flat, 200, OFFSET, 42, threads=1)
    assert np.array_equal(v, ov) and np.array_equal(g, og)


@pytest.mark.parametrize("seg", [1, 3, 4, 10])
def test_tangent_trip_lengths_with_tail(rocm, tapes, seg):
    """Tangent loop trips that do not divide the iteration count (C4 draws two
    normals per step, so odd trips are allowed)."""
    flat = tapes["C4"]
    opts = rocm.options("fp64", seg_len=seg, libm=1, mode=2)
    _, v, g = run_emulated(flat, opts, 64, rocm=rocm)
    ov, _ = oracle.replay_paths(flat, 64, OFFSET, 42, threads=1)
    assert_values_match(v, ov, rocm.lower(flat, opts))
    check_per_path(v, g, flat, 64, OFFSET, 42, min_strict=STRICT["C4"], max_above=ABOVE["C4"])


def test_unrolled_straight_line_matches(rocm, tapes):
    flat = equity_tape_flat = tapes["C2"]
    _, v, g = run_emulated(equity_tape_flat, rocm.options("fp64", roll=-1, libm=1, mode=1), 64, rocm=rocm)
    ov, og = oracle.replay_paths(flat, 64, OFFSET, 42, threads=1)
    assert np.array_equal(v, ov) and np.array_equal(g, og)
    _, v, g = run_emulated(equity_tape_flat, rocm.options("fp64", roll=-1, libm=1, mode=2), 64, rocm=rocm)
    assert np.array_equal(v, ov)
    check_per_path(v, g, flat, 64, OFFSET, 42, min_strict=STRICT["C2"], max_above=ABOVE["C2"])


def line_plan(src):
    """The checkpointed straight line's plan line of a generated kernel."""
    m = re.search(r"// checkpointed straight line: (\d+) segments of about (\d+) nodes, (\d+) values stored per path, "
                  r"(\d+) values and (\d+) adjoints carried", src)
    return None if m is None else dict(zip(("segments", "seg_len", "stored", "values", "adjoints"),
                                           map(int, m.groups())))


@pytest.mark.parametrize("which,seg", [("asian120", 48), ("asian120", 96), ("asian32", 17), ("branching", 19)])
def test_checkpointed_straight_line_is_bit_exact(nt, rocm, which, seg):
    """The reference's checkpoint parity cases (CudaCheckpointParityTest.java:61-85:
    Asian 120 fixings at 48 and 96 nodes per segment, Asian 32 at 17, the
    branching tape at 19), lowered without their step loop and swept in reverse
    segment by segment: with libm Box-Muller every value and adjoint equals the
    oracle's bit for bit (the rules run in the uncut sweep's order), for 513
    paths at a 32-bit-crossing offset, both of the reference's seeds, and a
    moved input."""
    from conftest import asian_tape, branching_tape
    tape = {"asian120": lambda: asian_tape(nt, 120), "asian32": lambda: asian_tape(nt, 32),
            "branching": lambda: branching_tape(nt)}[which]()
    flat = tape.flat()
    opts = rocm.options("fp64", roll=-1, mode=1, libm=1, seg_len=seg)
    src = rocm.lower(flat, opts)
    plan = line_plan(src)
    n = len(flat["op"])
    assert plan is not None and plan["seg_len"] == seg and plan["segments"] == -(-n // seg)
    k = emu.EmulatedKernel(src, len(flat["input_node"]), tape_slots(src))
    moved = list(flat["recorded_inputs"])
    moved[0] = {"asian120": 101.0, "asian32": 98.0, "branching": 1.5}[which]
    for seed in (42, 0x12345678FEDCBA98):
        for x in (flat["recorded_inputs"], moved):
            _, v, g = k.run(x, 513, OFFSET, seed, grid=3, block=64)
            ov, og = oracle.replay_paths(flat, 513, OFFSET, seed, inputs=x, threads=1)
            assert np.array_equal(v, ov) and np.array_equal(g, og), (seed, x[0])


def test_checkpointed_straight_line_plan(rocm, tapes):
    """The 252-fixing Asian lowered without its loop: sqrt(1536) < 48, so 32
    segments of about 48 nodes, each boundary moved to where the fewest values
    cross it. Each value a later segment's reverse reads is stored once (the
    two loop-invariant step coefficients and the one or two values that cross
    each boundary); four values and four adjoints are carried."""
    src = rocm.lower(tapes["C2"], rocm.options("fp64", roll=-1, mode=1))
    assert line_plan(src) == dict(segments=32, seg_len=48, stored=34, values=4, adjoints=4)
    assert tape_plan(src)["tape_slots"] == "34"
    # below 512 nodes, or with every value stored, no cut
    assert line_plan(rocm.lower(tapes["C1"], rocm.options("fp64", roll=-1, mode=1))) is None
    assert line_plan(rocm.lower(tapes["C2"], rocm.options("fp64", roll=-1, mode=1, checkpoint=3))) is None
    # tangent mode carries no tape
    assert line_plan(rocm.lower(tapes["C2"], rocm.options("fp64", roll=-1, mode=2))) is None


def test_checkpointed_straight_line_sinks_a_schedule(rocm):
    """The weekday-fixing Asian lowered without its loop: its step schedule
    (computed before the first step) would be carried across every boundary;
    moved next to the steps that read it, three values and three adjoints
    cross a boundary. Per path within the bar (the moved nodes accumulate the
    shared inputs' adjoints in another order)."""
    from nablatensor_amd import workloads
    flat = workloads.schedule_tapes()["asian_weekdays"].flat()
    opts = rocm.options("fp64", roll=-1, mode=1, libm=1)
    src = rocm.lower(flat, opts)
    assert line_plan(src) == dict(segments=53, seg_len=53, stored=54, values=3, adjoints=3)
    _, v, g = run_emulated(flat, opts, 200, rocm=rocm)
    ov, _ = oracle.replay_paths(flat, 200, OFFSET, 42, threads=1)
    assert np.array_equal(v, ov)
    check_per_path(v, g, flat, 200, OFFSET, 42, min_strict=0.95)


@pytest.mark.parametrize("seed,seg", [(0, 9), (1, 17), (2, 31), (3, 48)])
def test_checkpointed_straight_line_random_tapes(nt, rocm, seed, seg):
    """Random single-output tapes (two inputs, normals on two streams,
    uniforms, every operation) lowered without a loop and cut into short
    segments: with libm Box-Muller every value and adjoint equals the
    oracle's bit for bit."""
    from conftest import random_tape
    flat = random_tape(nt, 10 + seed, 80 + 70 * seed, outputs=1).flat()
    opts = rocm.options("fp64", roll=-1, mode=1, libm=1, seg_len=seg)
    src = rocm.lower(flat, opts)
    assert line_plan(src)["seg_len"] == seg
    k = emu.EmulatedKernel(src, len(flat["input_node"]), tape_slots(src))
    _, v, g = k.run(flat["recorded_inputs"], 300, OFFSET, 42, grid=3, block=64)
    ov, og = oracle.replay_paths(flat, 300, OFFSET, 42, threads=1)
    assert np.array_equal(v, ov) and np.array_equal(g, og)


@pytest.mark.parametrize("precision", ["fp64", "fp32"])
def test_checkpointed_straight_line_exception_kernel(nt, rocm, precision):
    """The Merton jump tape (its saturating indicator overflows exp on most
    paths) lowered without its loop and cut into 40-node segments: the
    exception kernel re-evaluates the flagged paths segment by segment with
    the oracle's zero-adjoint rule; no NaN, per path within the bar (fp64),
    sums within 1e-5 of the fp32 oracle (fp32)."""
    from conftest import merton_call_tape
    m = dict(spot=100.0, strike=100.0, vol=0.18, rate=0.03, maturity=1.0, jumpIntensity=0.75, jumpMean=-0.05,
             jumpVol=0.15)
    flat = merton_call_tape(nt, m, steps=32).flat()
    opts = rocm.options(precision, roll=-1, mode=1, seg_len=40)
    src = rocm.lower(flat, opts)
    assert line_plan(src)["seg_len"] == 40 and "void nt_replay_slow(" in src
    sums, v, g = run_emulated(flat, opts, 256, rocm=rocm)
    assert np.all(np.isfinite(sums)) and np.all(np.isfinite(g))
    if precision == "fp64":
        check_per_path(v, g, flat, 256, OFFSET, 42, min_strict=0.98)
    else:
        ref = oracle.replay_sums(flat, 256, OFFSET, 42, f32=True)
        assert rel_err(sums, ref, floor=1.0) <= 1e-5


def test_price_only_and_moved_inputs(rocm, tapes):
    """Price only, at inputs other than the recorded ones: by default in the
    tangent frame with no tangents (the frame several input sets per dispatch
    use), and with the reverse frame forced the step-by-step forward pass,
    bit-equal to the oracle."""
    flat = tapes["C3"]
    x = [95.0, 101.0, 0.3, 0.01, 0.75]
    ov, _ = oracle.replay_paths(flat, 200, OFFSET, 42, inputs=x, threads=1)
    assert _mode(rocm, flat, adjoints=False) == "tangent"
    opts = rocm.options("fp64", adjoints=False, libm=1)
    sums, v, _ = run_emulated(flat, opts, 200, inputs=x, rocm=rocm)
    assert_values_match(v, ov, rocm.lower(flat, opts))
    assert np.all(sums[2:] == 0.0)
    sums, v, _ = run_emulated(flat, rocm.options("fp64", adjoints=False, libm=1, mode=1), 200, inputs=x, rocm=rocm)
    assert np.array_equal(v, ov)
    assert np.all(sums[2:] == 0.0)


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("name", ["no_draws", "input_out", "const_out", "draw_out"])
def test_degenerate_tapes(rocm, nt, name, mode):
    """No draws, an output that is an input, a zero derivative, an output that
    is a draw: the oracle's values and derivatives bit for bit."""
    flat = degenerate_tapes(nt)[name]
    sums, v, g = run_emulated(flat, rocm.options("fp64", libm=1, mode=mode), 150, rocm=rocm)
    ov, og = oracle.replay_paths(flat, 150, OFFSET, 42, threads=1)
    assert np.array_equal(v, ov) and np.array_equal(g, og)
    assert rel_err(sums, oracle.replay_sums(flat, 150, OFFSET, 42, threads=1), floor=1e-300) <= 1e-13


@pytest.mark.parametrize("mode", [1, 2])
def test_tape_with_no_inputs(rocm, nt, mode):
    """A tape with no inputs lowers to a kernel with two channels (Σy, Σy²)
    and no derivative columns: the oracle's values bit for bit with libm
    draws, within 1e-12 with the skeleton's own math."""
    flat = no_input_tape(nt).flat()
    assert len(flat["input_node"]) == 0
    ov, og = oracle.replay_paths(flat, 500, OFFSET, 42, threads=1)
    ref = oracle.replay_sums(flat, 500, OFFSET, 42, threads=1)
    assert og.shape == (500, 0) and len(ref) == 2
    sums, v, g = run_emulated(flat, rocm.options("fp64", libm=1, mode=mode), 500, rocm=rocm)
    assert g.shape == (500, 0) and len(sums) == 2
    assert np.array_equal(v, ov)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-13
    sums, v, _ = run_emulated(flat, rocm.options("fp64", mode=mode), 500, rocm=rocm)
    assert rel_err(v, ov) <= 1e-12
    assert rel_err(sums, ref, floor=1e-300) <= 1e-12


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("name,paths", [("C1", 700), ("C2", 300), ("C3", 200), ("C4", 100), ("C5", 30)])
def test_emulated_own_math_within_1e12(rocm, tapes, name, paths, mode):
    """The skeleton's own log/sqrt/sincos keep paths within the per-path bar."""
    flat = tapes[name]
    _, v, g = run_emulated(flat, rocm.options("fp64", mode=mode), paths, rocm=rocm)
    check_per_path(v, g, flat, paths, OFFSET, 42, min_strict=STRICT[name], max_above=ABOVE[name])


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("name,paths", [("C2", 300), ("C3", 300), ("C5", 40)])
def test_emulated_fp32_tracks_fp32_oracle(rocm, tapes, name, paths, mode):
    flat = tapes[name]
    sums, v, g = run_emulated(flat, rocm.options("fp32", mode=mode), paths, rocm=rocm)
    ov, og = oracle.replay_paths(flat, paths, OFFSET, 42, f32=True, threads=1)
    assert rel_err(v, ov) < 2e-4
    assert rel_err(g, og) < 2e-3


def test_lookback_and_digital_tapes(nt, rocm):
    m = nt.EquityMarket.atmOneYear()
    for product in (nt.Products.lookbackCall(), nt.Products.lookbackPut(),
                    nt.ExoticProducts.digitalCash(nt.OptionTypeEnum.CALL, 1.0, 0.5),
                    nt.ExoticProducts.barrier(nt.OptionTypeEnum.PUT, nt.ExoticProducts.BarrierEnum.UP_OUT, 120.0, 2.0)):
        flat = equity_tape(nt, product, m, 24).flat()
        ov, og = oracle.replay_paths(flat, 96, OFFSET, 42, threads=1)
        for ckpt in (1, 2, 3):
            _, v, g = run_emulated(flat, rocm.options("fp64", checkpoint=ckpt, libm=1, mode=1), 96, rocm=rocm)
            assert np.array_equal(v, ov) and np.array_equal(g, og), (product.label, ckpt)
        opts = rocm.options("fp64", libm=1, mode=2)
        _, v, g = run_emulated(flat, opts, 96, rocm=rocm)
        assert_values_match(v, ov, rocm.lower(flat, opts))
        check_per_path(v, g, flat, 96, OFFSET, 42, min_strict=0.95)  # measured 0.958 on these tapes


def test_loop_plan_of_the_workloads(rocm, tapes):
    def plan(name, **kw):
        src = rocm.lower(tapes[name], rocm.options(**kw))
        head = src.splitlines()[1]
        return head
    assert "start 15, period 6, iterations 252, draws/iter 1" in plan("C2")
    assert "start 15, period 16, iterations 252, draws/iter 1" in plan("C3")
    assert "period 30, iterations 504, draws/iter 2" in plan("C4")
    assert "period 504, iterations 252, draws/iter 16" in plan("C5")
    assert "straight line" in rocm.lower(tapes["C1"], rocm.options()).splitlines()[0]


def test_draw_pairs_share_one_philox_block(rocm, tapes):
    for mode in (1, 2):
        src = rocm.lower(tapes["C2"], rocm.options("fp64", checkpoint=1, seg_len=14, mode=mode))
        fwd = src.split("for (nt_u32 sg = 0;")[1].split("nt_y[")[0]
        assert fwd.count("nt_normal_pair(") == 7  # 14 draws per segment, two legs per block


def tape_plan(src):
    head = [ln for ln in src.splitlines() if ln.startswith("// nt-plan:")][0]
    return dict(kv.split("=") for kv in head.split()[2:])


def _mode(rocm, flat, **kw):
    head = [ln for ln in rocm.lower(flat, rocm.options(**kw)).splitlines() if ln.startswith("// nt-plan:")][0]
    return dict(kv.split("=") for kv in head.split()[2:])["mode"]


def _product_chain(n):
    """y = x0 * x1 * ... * x(n-1): every node depends on all inputs before it."""
    op, a, b = [1] * n, list(range(n)), [-1] * n
    prev = 0
    for i in range(1, n):
        op.append(6)  # MUL
        a.append(prev)
        b.append(i)
        prev = len(op) - 1
    return {"op": np.array(op), "arg_a": np.array(a), "arg_b": np.array(b), "constant": np.zeros(len(op)),
            "input_node": np.arange(n), "output_node": np.array([prev]), "n_streams": 1, "n_uniforms": 0,
            "recorded_inputs": [1.0 + 0.01 * i for i in range(n)]}


def test_cost_model_picks_the_cheaper_mode(rocm, tapes):
    # A Monte-Carlo step loop whose state depends on few inputs: tangents are
    # cheaper than recomputing the step for the reverse sweep.
    assert _mode(rocm, tapes["C2"]) == "tangent"
    assert _mode(rocm, tapes["C2"], mode=1) == "reverse"
    # A product of 40 inputs: node k carries k tangents, the reverse sweep two
    # adjoint updates per node.
    chain = _product_chain(40)
    assert _mode(rocm, chain) == "reverse"
    assert _mode(rocm, chain, mode=2) == "tangent"
    # price only: the tangent frame with no tangents, unless the reverse frame is forced
    assert _mode(rocm, tapes["C2"], adjoints=False) == "tangent"
    assert _mode(rocm, tapes["C2"], adjoints=False, mode=1) == "reverse"


def test_product_chain_both_modes_match_oracle(rocm):
    flat = _product_chain(12)
    ov, og = oracle.replay_paths(flat, 8, 0, 1, threads=1)
    for mode in (1, 2):
        _, v, g = run_emulated(flat, rocm.options("fp64", mode=mode), 8, offset=0, seed=1, rocm=rocm)
        assert np.array_equal(v, ov)
        assert rel_err(g, og) <= 1e-15


def test_exp_outside_fast_range_falls_back_per_path(rocm):
    """y = exp(a z) with a = 300: paths with |z| > 2.36 put the exponent past
    708; they are evaluated again with libm exp (overflow to inf included) and
    agree with the oracle, the others take the table-driven exp."""
    flat = {"op": np.array([1, 2, 6, 9]), "arg_a": np.array([0, 0, 0, 2]), "arg_b": np.array([-1, 0, 1, -1]),
            "constant": np.zeros(4), "input_node": np.array([0]), "output_node": np.array([3]),
            "n_streams": 1, "n_uniforms": 0, "recorded_inputs": [300.0]}
    ov, og = oracle.replay_paths(flat, 3000, 0, 5, threads=1)
    beyond = np.abs(np.log(np.abs(ov) + 1e-300)) > 708  # the exponent's own size, from the oracle
    assert 10 < beyond.sum() < 300 and np.isinf(ov).any()
    for mode in (1, 2):
        # libm=2: own log/sqrt with libm sincos keeps the draws within an ulp or
        # two of glibc's, so an exponent of 300 z does not amplify them past the bar
        _, v, g = run_emulated(flat, rocm.options("fp64", mode=mode, libm=2), 3000, offset=0, seed=5, rocm=rocm)
        ev, eg = oracle.path_errors(v, g, ov, og)
        assert ev.max() <= 1e-12 and eg.max() <= 1e-12, mode
        assert np.array_equal(np.isinf(v), np.isinf(ov))
        fast = ~beyond & np.isfinite(ov)
        assert ev[fast].max() <= 1e-12


@pytest.mark.parametrize("a", [0.3, 300.0])
def test_loop_exponent_bound_checked_once_per_path(nt, rocm, a):
    """s exp(a z) per step: the tangent kernel bounds the exponents before the
    loop (|a| 6.77 <= 708) and the loop's exponentials skip their own check;
    with a = 300 every path fails the bound and is evaluated again with libm
    exp (overflow and underflow included), agreeing with the oracle."""
    flat = scaled_exp_tape(nt, a).flat()
    src = rocm.lower(flat, rocm.options("fp64", mode=2))
    assert "6.77 * fabs(" in src and "nt_exp_core(" in src
    ov, og = oracle.replay_paths(flat, 600, 0, 5, threads=1)
    if a > 1:
        assert np.isinf(ov).any() and (ov == 0).any()
    _, v, g = run_emulated(flat, rocm.options("fp64", mode=2, libm=2), 600, offset=0, seed=5, rocm=rocm)
    ev, eg = oracle.path_errors(v, g, ov, og)
    assert ev.max() <= 1e-12  # overflowed values agree as infinities, underflowed ones as zeros
    # derivatives of overflowing products depend on the order of the products
    # (reverse against forward accumulation); the finite paths are held to the bar
    finite = np.isfinite(ov) & np.isfinite(og).all(axis=1) & (np.abs(og) < 1e300).all(axis=1)
    assert finite.sum() > 100 and eg[finite].max() <= 1e-12


@pytest.mark.parametrize("s_val,floor", [(1e-3, True), (1e-310, True), (1e-3, False)])
def test_sqrt_fast_routine_and_its_fallback(nt, rocm, s_val, floor):
    """SQRT nodes of tangent kernels take nt_sqrt_q: +0 arguments (z <= 0
    under the floor) stay on it; subnormal arguments (s = 1e-310) and
    negative ones (no floor: NaN roots) flag the path, which is evaluated
    again with libm sqrt. Values and derivatives agree with the oracle,
    NaN for NaN."""
    flat = sqrt_classes_tape(nt, s_val, floor).flat()
    assert "nt_sqrt_q(" in rocm.lower(flat, rocm.options("fp64", mode=2))
    ov, og = oracle.replay_paths(flat, 300, 0, 9, threads=1)
    if not floor:
        assert np.isnan(ov).any()
    _, v, g = run_emulated(flat, rocm.options("fp64", mode=2), 300, offset=0, seed=9, rocm=rocm)
    ev, eg = oracle.path_errors(v, g, ov, og)
    assert ev.max() <= 1e-12 and eg.max() <= 1e-12
    assert np.array_equal(np.isnan(v), np.isnan(ov))


@pytest.mark.parametrize("name,paths", [("C2", 200), ("C4", 64)])
def test_markets_share_draws_and_match_single_market_bit_for_bit(rocm, tapes, name, paths):
    """A kernel pricing three input sets per path gives each set exactly the
    single-market kernel's per-path values, derivatives and sums."""
    flat = tapes[name]
    x0 = np.array(flat["recorded_inputs"])
    sets = np.stack([x0, x0 * 1.01, x0 * 0.97])
    src = rocm.lower(flat, rocm.options("fp64", markets=3))
    # the fast pass draws once per path, as a single-market kernel with the same trip length does
    one = rocm.lower(flat, rocm.options("fp64", mode=2, seg_len=int(tape_plan(src)["seg"])))
    fast = lambda text: text.split("void nt_replay_slow(")[0].count("nt_normal_pair(")  # the replay kernel alone
    assert fast(src) == fast(one) > 0
    k = emu.EmulatedKernel(src, len(x0), 0)
    sums, v, g = k.run(sets, paths, OFFSET, 42, grid=3, block=64, markets=3)
    for m in range(3):
        s1, v1, g1 = run_emulated(flat, rocm.options("fp64", mode=2), paths, inputs=sets[m], rocm=rocm)
        assert np.array_equal(v[m], v1) and np.array_equal(g[m], g1), m
        assert np.array_equal(sums[m], s1), m


def test_uniforms_and_named_streams_match_oracle(nt, rocm):
    """The reference's random-streams body (a named-stream uniform beside the
    default-stream normal each step): the reverse sweep equals the oracle bit
    for bit with libm Box-Muller, tangent mode in values bit for bit and in
    derivatives to the per-path bar, for a straight-line and a rolled tape."""
    from conftest import jump_clock_tape
    for steps, rolled in ((3, False), (64, True)):
        flat = jump_clock_tape(nt, steps).flat()
        src = rocm.lower(flat, rocm.options("fp64", mode=1, libm=1))
        assert ("rolled loop" in src) == rolled
        assert "rhi1 = rhi ^ 0x9E3779B1u" in src
        ov, og = oracle.replay_paths(flat, 300, OFFSET, 42, threads=1)
        _, v, g = run_emulated(flat, rocm.options("fp64", mode=1, libm=1), 300, rocm=rocm)
        assert np.array_equal(v, ov) and np.array_equal(g, og), steps
        _, v, g = run_emulated(flat, rocm.options("fp64", mode=2, libm=1), 300, rocm=rocm)
        assert np.array_equal(v, ov), steps
        check_per_path(v, g, flat, 300, OFFSET, 42)


def test_multi_output_rows_match_oracle(nt, rocm):
    """Two outputs: every output's per-path value and Jacobian row, and its
    sums, against the oracle's (which sweeps the outputs one by one)."""
    from conftest import two_output_tape
    flat = two_output_tape(nt).flat()
    src = rocm.lower(flat, rocm.options("fp64", libm=1))
    assert "mode=tangent" in src and "rolled loop" in src
    k = emu.EmulatedKernel(src, 3, tape_slots(src))
    sums, v, g = k.run(flat["recorded_inputs"], 200, OFFSET, 42, grid=3, block=64, outputs=2)
    ov, og = oracle.replay_paths(flat, 200, OFFSET, 42, threads=1, output=None)
    assert np.array_equal(v, ov)
    for o in range(2):
        ev, eg = oracle.path_errors(v[:, o], g[:, o, :], ov[:, o], og[:, o, :])
        assert ev.max() == 0.0 and eg.max() <= 1e-12, o
    ref = oracle.replay_sums(flat, 200, OFFSET, 42, threads=1, all_outputs=True).reshape(2, -1)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-12


def _growth_tape(nt, steps=24):
    """S <- S exp(0.2 vol z - 0.01) per step and a running sum of S: a carried
    value updated by a single-use exponential, read by a sum."""
    def body(rec):
        s0 = rec.input("S0", 100.0)
        vol = rec.input("vol", 0.3)
        s = s0
        acc = rec.constant(0.0)
        for _ in range(steps):
            s = s.mul(vol.mul(rec.randn()).mul(0.2).sub(0.01).exp())
            acc = acc.add(s)
        rec.output(acc.mul(0.5).add(s))
    return nt.AadRecorder.record(body).flat()


@pytest.mark.parametrize("precision", ["fp64", "fp32"])
def test_multiplicative_carry_tangents(nt, rocm, precision):
    """Tangent mode carries such a value's tangent as G sigma (G the product of
    the exponentials since the loop began, sigma = t(start) + c0 sum tx): no
    division, so a start value of zero (where the tangent is still G t(start),
    not zero) is exact too."""
    flat = _growth_tape(nt)
    src = rocm.lower(flat, rocm.options(precision, mode=2))
    assert "real gs" in src and "c0_" in src
    for s0 in (100.0, 0.0):
        x = [s0, 0.3]
        ov, og = oracle.replay_paths(flat, 64, OFFSET, 9, inputs=x, threads=1)
        _, v, g = run_emulated(flat, rocm.options(precision, mode=2, libm=1), 64, seed=9, inputs=x, rocm=rocm)
        if precision == "fp64":
            ev, eg = oracle.path_errors(v, g, ov, og)
            assert ev.max() <= 1e-13 and eg.max() <= 1e-12, s0
        else:
            assert rel_err(g, og) <= 1e-4, s0
        if s0 == 0.0:
            assert np.all(v == 0.0) and np.all(np.abs(og[:, 0]) > 0.1) and np.all(og[:, 1] == 0.0)


def test_multiplicative_carries_only_where_they_pay(nt, rocm, tapes):
    """The Asian spot (read by a sum), the Heston spot, the 16 worst-of spots
    (read only after the loop) and both barrier carries (the spot, read by
    the smoothed barrier test through scalings, and the survival product, a
    carry times 1 / (1 + e)) take G sigma. A carry multiplied by another
    value with a tangent keeps the product rule (below)."""
    def carries(src):  # distinct G-form carries (the re-evaluation pass declares its own copies)
        return len(set(re.findall(r"real (gs\d+) ", src)))
    gs = {k: carries(rocm.lower(tapes[k], rocm.options("fp32", mode=2))) for k in ("C2", "C3", "C4", "C5")}
    assert gs == {"C2": 1, "C3": 2, "C4": 1, "C5": 16}

    def body(rec):
        s = rec.input("S0", 100.0)
        vol = rec.input("sigma", 0.2)
        acc = s.mul(0.0)
        for _ in range(16):
            s = s.mul(vol.mul(rec.randn()).exp())
            acc = acc.add(s.mul(vol))  # a product with a value that has a tangent for sigma
        rec.output(acc)
    flat = nt.AadRecorder.record(body).flat()
    assert carries(rocm.lower(flat, rocm.options("fp64", mode=2))) == 0


@pytest.mark.parametrize("name,paths", [("C2", 300), ("C3", 200), ("C4", 100), ("C5", 30)])
def test_loop_tangents_over_parameters_or_inputs(rocm, tapes, name, paths):
    """The step loop's tangents run over the loop's parameters (the
    loop-invariant values the step reads, the carries' start values) and go
    back to the inputs once per path after the loop, or run over the inputs
    directly: the same values bit for bit, derivatives within the per-path
    bar of the oracle in both, and within 1e-12 of each other."""
    flat = tapes[name]
    ov, og = oracle.replay_paths(flat, paths, OFFSET, 42, threads=1)
    grads = {}
    for basis in (1, 2):
        opts = rocm.options("fp64", libm=1, mode=2, basis=basis)
        src = rocm.lower(flat, opts)
        assert tape_plan(src)["basis"] == ("inputs" if basis == 1 else "params")
        _, v, g = run_emulated(flat, opts, paths, rocm=rocm)
        assert_values_match(v, ov, src)
        check_per_path(v, g, flat, paths, OFFSET, 42, min_strict=STRICT[name], max_above=ABOVE[name])
        grads[basis] = g
    assert rel_err(grads[2], grads[1]) <= 1e-12


def test_loop_basis_chosen_by_tangents_per_step(rocm, tapes):
    """The engine runs the loop over parameters where that makes fewer
    tangents per step (the Asian step: drift and volatility against r,
    sigma and T; the barrier), in fp32 also where it makes as many (the
    worst-of basket), and over the inputs where the parameters outnumber
    them (Heston's step reads more invariant values than it has inputs)."""
    plan = {k: tape_plan(rocm.lower(tapes[k], rocm.options("fp64", mode=2))) for k in ("C2", "C3", "C4", "C5")}
    assert {k: v["basis"] for k, v in plan.items()} == {"C2": "params", "C3": "params", "C4": "inputs", "C5": "inputs"}
    assert tape_plan(rocm.lower(tapes["C5"], rocm.options("fp32", mode=2)))["basis"] == "params"
    assert plan["C2"]["params"] == "3"  # drift, volatility, the spot's start value


def _shared_parameter_tape(nt):
    """The start value of the carried spot is also read by every step (a
    floor proportional to it): one parameter for both, whose tangent for
    itself is 1 in both roles."""
    def body(rec):
        s0 = rec.input("S0", 100.0)
        vol = rec.input("sigma", 0.25)
        k = rec.input("K", 98.0)
        x = s0
        acc = s0.mul(0.0)
        for _ in range(16):
            x = x.mul(vol.mul(rec.randn()).exp()).max(s0.mul(0.8))
            acc = acc.add(x.sub(k).max(0.0))
        rec.output(acc)
    return nt.AadRecorder.record(body).flat()


def test_parameter_read_both_as_start_value_and_in_the_step(nt, rocm):
    flat = _shared_parameter_tape(nt)
    src = rocm.lower(flat, rocm.options("fp64", mode=2, basis=2))
    # S0 (the spot's start value, and read by the floor's product), sigma, K,
    # and the sum's start value S0 * 0 (a node of its own)
    assert tape_plan(src)["params"] == "4"
    ov, og = oracle.replay_paths(flat, 256, OFFSET, 5, threads=1)
    for basis in (1, 2):
        _, v, g = run_emulated(flat, rocm.options("fp64", mode=2, libm=1, basis=basis), 256, seed=5, rocm=rocm)
        ev, eg = oracle.path_errors(v, g, ov, og)
        assert ev.max() <= 1e-13 and eg.max() <= 1e-12, basis
    assert np.any(og[:, 0] != 0.0) and np.any(og[:, 2] != 0.0)


def test_exponent_fused_only_for_a_carry_kept_as_g(nt, rocm, tapes):
    """drift + vol z feeding the Asian spot's factor is one fma (the spot is
    carried as G, its sum as the sum of G); a spot read every step as a value
    (the product of steps, as the oracle rounds it) keeps the rounded sum, and
    so does the device-libm kernel."""
    fused = re.compile(r"const real r\d+_\d+ = fma\(v\d+, r\d+_\d+, v\d+\);")
    assert len(fused.findall(rocm.lower(tapes["C2"], rocm.options("fp64", mode=2)))) > 0
    assert not fused.search(rocm.lower(tapes["C2"], rocm.options("fp64", mode=2, libm=1)))

    def body(rec):
        s = rec.input("S0", 100.0)
        mu = rec.input("mu", 0.001)
        vol = rec.input("sigma", 0.02)
        hi = s.mul(0.0)
        for _ in range(16):
            s = s.mul(mu.add(vol.mul(rec.randn())).exp())
            hi = hi.max(s)  # reads the spot's value every step
        rec.output(hi)
    flat = nt.AadRecorder.record(body).flat()
    src = rocm.lower(flat, rocm.options("fp64", mode=2))
    assert not fused.search(src)
    _, v, g = run_emulated(flat, rocm.options("fp64", mode=2), 256, seed=3, rocm=rocm)
    check_per_path(v, g, flat, 256, OFFSET, 3, min_strict=0.99)  # measured 0.996


def test_parameter_basis_on_assorted_tapes(nt, rocm):
    """The loop's tangents forced over parameters on tapes of other shapes
    (lookback and digital payoffs, an up-and-out barrier, a named-stream
    uniform beside the normal, two outputs, a carry read by a sum and by the
    payoff): values as the oracle's, derivatives to the per-path bar, every
    output's row."""
    from conftest import jump_clock_tape, two_output_tape
    m = nt.EquityMarket.atmOneYear()
    flats = [equity_tape(nt, p, m, 24).flat() for p in (
        nt.Products.lookbackCall(), nt.ExoticProducts.digitalCash(nt.OptionTypeEnum.CALL, 1.0, 0.5),
        nt.ExoticProducts.barrier(nt.OptionTypeEnum.PUT, nt.ExoticProducts.BarrierEnum.UP_OUT, 120.0, 2.0))]
    flats += [jump_clock_tape(nt, 64).flat(), _growth_tape(nt)]
    for flat in flats:
        opts = rocm.options("fp64", libm=1, mode=2, basis=2)
        src = rocm.lower(flat, opts)
        assert "rolled loop" in src and "basis=params" in src
        ov, _ = oracle.replay_paths(flat, 128, OFFSET, 42, threads=1)
        _, v, g = run_emulated(flat, opts, 128, rocm=rocm)
        assert_values_match(v, ov, src)
        check_per_path(v, g, flat, 128, OFFSET, 42, min_strict=0.93)  # measured 0.9375 on these tapes
    flat = two_output_tape(nt).flat()
    src = rocm.lower(flat, rocm.options("fp64", libm=1, basis=2))
    assert "basis=params" in src
    k = emu.EmulatedKernel(src, 3, tape_slots(src))
    _, v, g = k.run(flat["recorded_inputs"], 200, OFFSET, 42, grid=3, block=64, outputs=2)
    ov, og = oracle.replay_paths(flat, 200, OFFSET, 42, threads=1, output=None)
    assert np.array_equal(v, ov)
    for o in range(2):
        _, eg = oracle.path_errors(v[:, o], g[:, o, :], ov[:, o], og[:, o, :])
        assert eg.max() <= 1e-12, o


@pytest.mark.parametrize("name", ["C2", "C5"])
@pytest.mark.parametrize("precision", ["fp64", "fp32"])
def test_contract_off_emits_no_fused_node_value(tapes, precision, name):
    """contract=-1 keeps every product and sum of a tape node separately
    rounded: the fused exponent of a G-carried step factor and the worst-of's
    correlated normals (explicit fmas in the default kernel) become rounded
    products and sums again, and the worst-of's spots sum their exponents
    step by step instead of their normals."""
    from nablatensor_amd import rocm
    fused = re.compile(r"const real r\d+_\d+\w* = .*fmaf?\(")
    default = rocm.lower(tapes[name], rocm.options(precision))
    off = rocm.lower(tapes[name], rocm.options(precision, contract=-1))
    assert any(fused.search(line) for line in default.splitlines())
    assert not any(fused.search(line) for line in off.splitlines())
    assert "#pragma clang fp contract(off)" in off
    assert ("zq0_" in default) == (name == "C5") and "zq0_" not in off


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("precision,libm", [("fp64", 0), ("fp64", 1), ("fp32", 0)])
def test_saturating_indicator_follows_the_zero_adjoint_rule(nt, rocm, precision, libm, mode):
    """The Merton jump tape's smoothed indicator 1 / (1 + exp(-(lambda dt - u) /
    2e-4)) saturates on most steps: exp overflows to infinity and the
    indicator is exactly 0. The oracle never multiplies by a zero adjoint
    (ScalarReplay.java:134-136), so no derivative flows back through the
    overflowed exponential; IEEE arithmetic gives 0 x inf = NaN there in both
    derivative modes. Such paths go to the exception kernel, which keeps the
    oracle's rule: per path within the bar (fp64), the sums within 1e-5 of the
    fp32 oracle's (fp32), no NaN anywhere."""
    from conftest import merton_call_tape
    m = dict(spot=100.0, strike=100.0, vol=0.18, rate=0.03, maturity=1.0, jumpIntensity=0.75, jumpMean=-0.05,
             jumpVol=0.15)
    flat = merton_call_tape(nt, m, steps=32).flat()
    src = rocm.lower(flat, rocm.options(precision, mode=mode, libm=libm))
    assert "void nt_replay_slow(" in src
    sums, v, g = run_emulated(flat, rocm.options(precision, mode=mode, libm=libm), 256, rocm=rocm)
    assert np.all(np.isfinite(sums)) and np.all(np.isfinite(g))
    if precision == "fp64":
        check_per_path(v, g, flat, 256, OFFSET, 42, min_strict=0.98)  # measured 0.988
    else:
        ref = oracle.replay_sums(flat, 256, OFFSET, 42, f32=True)
        assert rel_err(sums, ref, floor=1.0) <= 1e-5


def test_step_schedule_recorded_up_front_rolls(rocm):
    """An Asian call on TimeGrid.of 252 weekday fixings records every step's
    drift and diffusion before the first step (GbmPath.java:61-66), with
    year fractions that differ in their last bits: moved next to the steps
    that read them, with the fractions read from a per-step table, the step
    repeats (11 nodes x 251 steps; the first step carries the shared
    half-variance and stays straight-line). Both modes compile in seconds
    with no scratch, where the straight-line kernel took two minutes of hipRTC
    and spilled 11-20 KB per lane."""
    from nablatensor_amd import workloads
    import time
    flat = workloads.schedule_tapes()["asian_weekdays"].flat()
    assert len(flat["op"]) == 2791
    for precision in ("fp64", "fp32"):
        for mode in (rocm.NT_MODE_REVERSE, rocm.NT_MODE_TANGENT):
            t0 = time.time()
            info = rocm.compile_check(flat, rocm.options(precision, mode=mode))
            assert (info["loop_period"], info["loop_iters"]) == (11, 251)
            assert info["scratch_bytes"] == 0
            assert time.time() - t0 < 60
    src = rocm.lower(flat, rocm.options("fp64"))
    assert src.count("__constant__ real nt_lit") == 1  # the step's year fraction


@pytest.mark.parametrize("mode,libm", [(1, 0), (1, 1), (2, 0), (2, 1)])
def test_step_schedule_per_path_matches_oracle(rocm, mode, libm):
    """The rolled weekday-fixing Asian against the oracle, per path (the
    reordered tape accumulates the adjoints of the schedule's shared inputs in
    another order, so the reverse sweep with libm is within the bar rather
    than bit-exact)."""
    from nablatensor_amd import workloads
    flat = workloads.schedule_tapes()["asian_weekdays"].flat()
    sums, v, g = run_emulated(flat, rocm.options("fp64", mode=mode, libm=libm), 300, rocm=rocm)
    ov, _ = oracle.replay_paths(flat, 300, OFFSET, 42, threads=1)
    assert np.array_equal(v, ov) or rel_err(v, ov) <= 1e-12
    check_per_path(v, g, flat, 300, OFFSET, 42, min_strict=0.95)  # measured 0.953
    ref = oracle.replay_sums(flat, 300, OFFSET, 42, threads=1)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-12


def test_uniform_workloads_keep_their_exact_loops(rocm, tapes):
    """Only a tape whose exactly repeating step covers less than half of it is
    reordered: the five workloads keep their plans (their sources are pinned
    by tests/golden/tape_digests.json), with no literal tables."""
    for name in ("C2", "C3", "C4", "C5"):
        assert "nt_lit" not in rocm.lower(tapes[name], rocm.options("fp64"))


@pytest.mark.parametrize("name,slots", [("C2", 18), ("C3", 84), ("C4", 336)])
def test_reverse_checkpoints_only_what_the_recompute_reads(rocm, tapes, name, slots):
    """A segment's recompute produces only the values its rules read and what
    they are computed from, so only the carries it reads are checkpointed: the
    Asian's running sum (read by no rule, its adjoint flows through additions)
    is not, leaving one slot per segment for the spot (C2: 18 segments of 14
    steps), two for the barrier and two of Heston's three carries."""
    src = rocm.lower(tapes[name], rocm.options("fp64", mode=1))
    plan = tape_plan(src)
    assert int(plan["tape_slots"]) == slots, plan


def test_step_schedule_computed_once_per_block_and_pairs_aligned(rocm, tapes):
    """The weekday Asian's tangent kernel computes the step schedule (drift and
    volatility per step, with their tangents over the inputs: 7 rows) once per
    block, so its step loop takes no square root; and since its loop's draws
    start at ordinal 1 (the first step is recorded before the loop), the loop
    runs its first step alone and then trips of two steps from step 1, each
    trip one whole Box-Muller pair. The uniform Asian (draws from ordinal 0,
    no schedule) keeps trips from step 0."""
    from nablatensor_amd import workloads
    flat = workloads.schedule_tapes()["asian_weekdays"].flat()
    src = rocm.lower(flat, rocm.options("fp64", mode=2))
    assert tape_plan(src)["schedule"] == "7"
    fast = src[:src.index("nt_replay_slow")]
    loop = fast[fast.index("for (nt_u32 sg = 0; sg < 125u; ++sg)"):]
    loop = loop[:loop.index("\n    }\n")]  # the trip's block
    assert "it0 = 1u + (sg) * 2u" in loop and "kb0 = it0 * 1u + 1u" in loop
    assert loop.count("nt_normal_pair(") == 1
    assert "sqrt" not in loop
    c2 = rocm.lower(tapes["C2"], rocm.options("fp64", mode=2))
    assert tape_plan(c2)["schedule"] == "0" and "it0 = 1u +" not in c2


def test_exp_factor_carries_sum_their_exponents(rocm, tapes):
    """A carry kept as G alone whose factor is exp(p + r s), p and r
    loop-invariant and s a correlated normal (the worst-of's 16 spots), adds s
    alone each step (zq = zs + s); after the loop the exponents' sum is
    N p + r S and one exponential follows, in the fast pass only. Without the
    static bound on s (device libm) the fp64 kernel adds the exponents
    themselves (gq = gs + x). A carry whose G is read every step (the Asian
    spot, summed into the average) keeps the product, and so does the
    barrier's survival product (its factor is 1 / b, not an exponential)."""
    for prec in ("fp64", "fp32"):
        src = rocm.lower(tapes["C5"], rocm.options(prec, mode=2))
        fast = src[:src.index("nt_replay_slow")]
        summed = set(re.findall(r"real zq0_(\d+) = zs\1 \+ r0_\d+;", fast))
        assert len(summed) == 16, prec
        assert not re.search(r"real gq0_\d+ = gs\d+ \+ ", fast)
        exp_after = r"nt_hw_exp2f\(gs{0}\)" if prec == "fp32" else r"nt_exp_fast\(gs{0}, nt_slow\)"
        fma = "fmaf" if prec == "fp32" else "fma"
        for j in summed:
            assert re.search(r"gs{0} = {1}\(\S+, zs{0}, \(0x1\.f8p\+7f?\) \* \S+\);".format(j, fma), fast), (prec, j)
            assert re.search(r"gs{0} = ".format(j) + exp_after.format(j), fast), (prec, j)
        slow = src[src.index("nt_replay_slow"):]
        assert not re.search(r"real (gq|zq)0_\d+ = (gs|zs)\d+ \+ ", slow)
    src = rocm.lower(tapes["C5"], rocm.options("fp64", mode=2, libm=1))
    fast = src[:src.index("nt_replay_slow")]
    assert len(set(re.findall(r"real gq0_(\d+) = gs\1 \+ ", fast))) == 16 and "zq0_" not in fast
    for name in ("C2", "C3", "C4"):
        src = rocm.lower(tapes[name], rocm.options("fp64", mode=2))
        assert not re.search(r"real (gq|zq)0_\d+ = (gs|zs)\d+ \+ ", src), name


@pytest.mark.parametrize("fixings", [63, 64])
@pytest.mark.parametrize("libm", [0, 1])
def test_weekday_grids_with_a_lead_step_and_tails(rocm, nt, fixings, libm):
    """Asian calls on weekday grids of 63 and 64 fixings: the loop's draws
    start at ordinal 1, so the tangent kernel runs the first loop step alone,
    then trips of two steps (61 steps after the lead: a tail trip of one; 62:
    none), with the step schedule computed once per block. Per path within the
    oracle's bar, sums within 1e-12."""
    from nablatensor_amd import workloads
    grid = nt.TimeGrid.of(workloads.weekday_fixings(fixings))
    flat = nt.record(nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), grid).flat()
    src = rocm.lower(flat, rocm.options("fp64", mode=2, libm=libm))
    assert "it0 = 1u + (sg) * 2u" in src and int(tape_plan(src)["schedule"]) > 0
    sums, v, g = run_emulated(flat, rocm.options("fp64", mode=2, libm=libm), 200, rocm=rocm)
    check_per_path(v, g, flat, 200, OFFSET, 42, min_strict=0.9)
    ref = oracle.replay_sums(flat, 200, OFFSET, 42, threads=1)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-12


def test_discounted_weekday_asian_reads_its_growth_from_the_schedule(rocm, nt):
    """A bank account growing by exp(r dt_i) on a weekday grid, read by the
    average every step: its factor is a schedule value (with its tangents for
    r and T) computed once per block; per path within the oracle's bar."""
    from conftest import discounted_weekday_asian_tape
    flat = discounted_weekday_asian_tape(nt, 48)
    src = rocm.lower(flat, rocm.options("fp64", mode=2))
    plan = tape_plan(src)
    assert plan["mode"] == "tangent" and int(plan["schedule"]) >= 10, plan
    for libm in (0, 1):
        sums, v, g = run_emulated(flat, rocm.options("fp64", mode=2, libm=libm), 150, rocm=rocm)
        check_per_path(v, g, flat, 150, OFFSET, 42, min_strict=0.85)  # measured 0.873
        # (the rate's pathwise sensitivity of a discounted average nearly cancels: floor 1)
        assert rel_err(sums, oracle.replay_sums(flat, 150, OFFSET, 42, threads=1), floor=1.0) <= 1e-12


@pytest.mark.parametrize("precision", ["fp64", "fp32"])
def test_signed_affine_exponents_summed_after_the_loop(rocm, nt, precision):
    """Spots whose step exponents are p - r w (w a correlated normal), r z - p
    and r z: each step adds its draw alone and N p + r S, with the signs, and
    the tangents follow the loop (fp32: exponents folded into exp2, in log2
    units). Per path within the bar of the oracle (fp64, own math), within
    fp32 rounding of the fp32 oracle."""
    from conftest import signed_basket_tape
    flat = signed_basket_tape(nt, 40)
    src = rocm.lower(flat, rocm.options(precision, mode=2))
    fast = src[:src.index("nt_replay_slow")]
    summed = len(set(re.findall(r"real zq0_(\d+) = zs\1 \+ ", fast)))
    assert summed == 3, precision
    fma, n, l2e = ("fma", r"\(0x1\.4p\+5\)", "") if precision == "fp64" else ("fmaf", r"\(0x1\.4p\+5f\)", "_l2e")
    assert re.search(r"gs\d+ = {0}\(-v\d+{2}, zs\d+, {1} \* v\d+{2}\);".format(fma, n, l2e), fast)
    assert re.search(r"gs\d+ = {0}\(v\d+{2}, zs\d+, {1} \* -v\d+{2}\);".format(fma, n, l2e), fast)
    assert re.search(r"gs\d+ = v\d+(_l2e)? \* zs\d+;", fast)
    _, v, g = run_emulated(flat, rocm.options(precision, mode=2), 200, rocm=rocm)
    if precision == "fp64":
        check_per_path(v, g, flat, 200, OFFSET, 42, min_strict=0.9)
    else:
        ov, og = oracle.replay_paths(flat, 200, OFFSET, 42, f32=True, threads=1)
        assert rel_err(v, ov) < 2e-4 and rel_err(g, og) < 2e-3


@pytest.mark.parametrize("k", [2, 8, 16])
def test_local_vol_tape_both_modes_emulated(rocm, k):
    """The parametric local-volatility Asian (workloads.local_vol_asian_tape):
    the cost model picks tangent mode for few coefficients and the reverse
    sweep from 12 on (the crossover measured on MI355X); both modes match the
    oracle, the reverse sweep bit for bit with libm Box-Muller, tangent mode
    within the per-path bar."""
    from nablatensor_amd import workloads
    flat = workloads.local_vol_asian_tape(k, steps=24).flat()
    auto = rocm.lower(flat, rocm.options("fp64"))
    assert ("mode=reverse" in auto) == (k >= 12)
    paths = 96
    ov, og = oracle.replay_paths(flat, paths, OFFSET, 42, threads=1)
    _, v, g = run_emulated(flat, rocm.options("fp64", libm=1, mode=1), paths, rocm=rocm)
    assert np.array_equal(v, ov) and np.array_equal(g, og)
    opts = rocm.options("fp64", libm=1, mode=2)
    _, v, g = run_emulated(flat, opts, paths, rocm=rocm)
    assert_values_match(v, ov, rocm.lower(flat, opts))
    check_per_path(v, g, flat, paths, OFFSET, 42, min_strict=0.9)


@pytest.mark.parametrize("mode", [1, 2])
def test_max_min_follow_java_math_emulated(nt, rocm, mode):
    """The fp64 fast pass's MAX and MIN (v_max_f64 with a NaN-making term, the
    exception kernel's exact rule behind it) per path against the oracle on
    signed zeros, NaN and infinities: tangent mode on the six-output tape, the
    reverse sweep on each output alone."""
    from conftest import MAX_MIN_CASES, MAX_MIN_OUTPUTS, max_min_tape, same_special
    tapes_ = [max_min_tape(nt).flat()] if mode == 2 else [max_min_tape(nt, o).flat() for o in range(MAX_MIN_OUTPUTS)]
    for flat in tapes_:
        opts = rocm.options("fp64", mode=mode)
        src = rocm.lower(flat, opts)
        assert ("nt_max_lit(" in src or "nt_min_lit(" in src or "nt_max_fast(" in src or "nt_min_fast(" in src)
        assert "nt_replay_slow" in src
        outputs = len(flat["output_node"])
        k = emu.EmulatedKernel(src, len(flat["input_node"]), tape_slots(src))
        for case in MAX_MIN_CASES:
            _, v, _ = k.run(list(case), 64, 0, 42, grid=3, block=64, outputs=outputs)
            ov, _ = oracle.replay_paths(flat, 64, 0, 42, inputs=list(case), threads=1, output=None)
            assert same_special(np.reshape(v, ov.shape), ov), (case, v[:1], ov[:1])


@pytest.mark.parametrize("mode", [1, 2])
def test_special_values_follow_the_oracle_emulated(nt, rocm, mode):
    """EXP, LOG, SQRT, DIV, 1 / x, ABS, NEG and MUL at signed zeros,
    subnormals, infinities, NaN and the exponential's overflow and underflow,
    per path against the oracle: the fast pass's own math flags what it does
    not cover and the exception kernel evaluates it with libm."""
    from conftest import SPECIAL_CASES, SPECIAL_OUTPUTS, close_special, special_ops_tape
    tapes_ = [special_ops_tape(nt).flat()] if mode == 2 else [special_ops_tape(nt, o).flat() for o in range(SPECIAL_OUTPUTS)]
    for flat in tapes_:
        src = rocm.lower(flat, rocm.options("fp64", mode=mode))
        k = emu.EmulatedKernel(src, len(flat["input_node"]), tape_slots(src))
        for case in SPECIAL_CASES:
            _, v, g = k.run(list(case), 64, 0, 42, grid=3, block=64, outputs=len(flat["output_node"]))
            ov, og = oracle.replay_paths(flat, 64, 0, 42, inputs=list(case), threads=1, output=None)
            assert close_special(np.reshape(v, ov.shape), ov, 4e-16), (case, flat["output_node"], v[:1], ov[:1])
            if mode == 1:
                # the reverse sweep's adjoints, special values included (tangent mode caps sqrt's
                # infinite derivative at 0 and can differ in the sign of a zero derivative)
                assert close_special(np.reshape(g, og.shape), og, 4e-16), (case, flat["output_node"], g[:1], og[:1])
