"""GPU parity of the HIP replay engine against the CPU oracle, through the C ABI.

Both derivative modes (the reverse sweep under each checkpoint policy, and
tangent mode) are held to the same bars. Bars (fp64): per path and per
component (the value and each Greek, relative with floor 1) within
max(1e-12, 8 x the oracle's own sensitivity to one-unit moves of its
transcendental results) (conftest.check_per_path), with the fraction of paths
held to 1e-12 itself pinned; sums over paths within 1e-10. fp32 reconciles with
the fp64 oracle within 1e-5 relative on price and on each first-order Greek
(conftest.reconcile). The reference-held aggregates of the Asian call
(docs/validation.md:56-63) are reproduced at their printed precision.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import ABOVE, STRICT, check_per_path, degenerate_tapes, no_input_tape, reconcile, rel_err

pytestmark = pytest.mark.gpu

OFFSET = 0x100000003  # crosses the 32-bit boundary of the Philox counter words


@pytest.fixture(scope="module")
def rocm():
    from nablatensor_amd import rocm as r
    assert r.probe() > 0, "no gfx950 device visible to libnt_rocm.so"
    return r


def test_device_is_gfx950(rocm):
    name, arch = rocm.device_name()
    assert arch.startswith("gfx950"), (name, arch)


# (derivative mode, checkpoint policy): the reverse sweep under each policy, and tangent mode
VARIANTS = [(1, 1), (1, 2), (1, 3), (2, 0)]


@pytest.mark.parametrize("libm", [0, 1])
@pytest.mark.parametrize("mode,ckpt", VARIANTS)
@pytest.mark.parametrize("name,paths", [("C1", 4096), ("C2", 2048), ("C3", 1024), ("C4", 512)])
def test_per_path_fp64_matches_oracle(rocm, tapes, name, paths, mode, ckpt, libm):
    t = tapes[name]
    print(f"case {name} mode={mode} ckpt={ckpt} libm={libm} paths={paths}", flush=True)
    with rocm.Executable(t, rocm.options("fp64", checkpoint=ckpt, libm=libm, mode=mode)) as x:
        v, g = x.replay_paths(paths, OFFSET, 42)
        info = x.info()
    assert info["scratch_bytes"] == 0
    assert info["mode"] == mode
    summary = check_per_path(v, g, t, paths, OFFSET, 42, min_strict=STRICT[name], max_above=ABOVE[name])
    print(summary)


@pytest.mark.parametrize("mode", [1, 2])
def test_per_path_fp64_heston_many_paths(rocm, tapes, mode):
    """4096 Heston paths: the sensitivity-scaled bound holds on every path and component."""
    t = tapes["C4"]
    print(f"case C4 mode={mode} paths=4096 seed=7", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        v, g = x.replay_paths(4096, OFFSET, 7)
    print(check_per_path(v, g, t, 4096, OFFSET, 7, min_strict=STRICT["C4"], max_above=ABOVE["C4"]))


@pytest.mark.parametrize("mode", [1, 2])
def test_per_path_fp64_worst_of_matches_oracle(rocm, tapes, mode):
    """The worst-of per path in both modes; its fp64 tangent kernel is the one
    compiled again for two waves per SIMD (at most 256 VGPRs, no scratch)."""
    t = tapes["C5"]
    print(f"case C5 mode={mode} paths=256", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        v, g = x.replay_paths(256, 7, 42)
        info = x.info()
        if mode == 2:
            assert info["vgprs"] <= 256 and info["scratch_bytes"] == 0, info
            assert "__launch_bounds__(256, 2)" in x.source()
    print(check_per_path(v, g, t, 256, 7, 42, min_strict=STRICT["C5"], max_above=ABOVE["C5"]))


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("name,paths", [("C1", 1_000_000), ("C2", 200_000), ("C3", 100_000)])
def test_sums_fp64_match_oracle(rocm, tapes, name, paths, mode):
    t = tapes[name]
    print(f"case {name} mode={mode} paths={paths}", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        sums, _ = x.replay(paths, 0, 42)
    ref = oracle.replay_sums(t, paths, 0, 42)
    assert rel_err(sums[[0] + list(range(2, len(sums)))], ref[[0] + list(range(2, len(ref)))], floor=1e-300) <= 1e-10
    assert abs(sums[1] - ref[1]) <= 1e-10 * abs(ref[1])


@pytest.mark.parametrize("mode", [1, 2])
def test_published_asian_aggregates(rocm, tapes, mode):
    """Asian call, 252 fixings, ATM 1y, fp64, seed 42, 1,000,000 scenarios:
    the oracle values printed in the reference's evidence pack."""
    with rocm.Executable(tapes["C2"], rocm.options("fp64", mode=mode)) as x:
        sums, _ = x.replay(1_000_000, 0, 42)
    r = oracle.to_result(sums, 1_000_000)
    published = {"price": 5.3058639800, "delta": 0.56198939096, "dK": -0.50893075116, "vega": 22.412432861,
                 "rho": 23.603384920, "dT": 2.9493448337}
    got = {"price": r["price"], "delta": r["gradient"][0], "dK": r["gradient"][1], "vega": r["gradient"][2],
           "rho": r["gradient"][3], "dT": r["gradient"][4]}
    for k, ref in published.items():
        assert abs(got[k] - ref) <= 5e-11 * abs(ref), (k, got[k], ref)


@pytest.mark.parametrize("mode", [1, 2])
@pytest.mark.parametrize("name,paths", [("C2", 200_000), ("C3", 100_000)])
def test_fp32_reconciles_with_fp64_oracle(rocm, tapes, name, paths, mode):
    t = tapes[name]
    with rocm.Executable(t, rocm.options("fp32", mode=mode)) as x:
        sums, _ = x.replay(paths, 0, 42)
    ref = oracle.replay_sums(t, paths, 0, 42)
    errs = reconcile(sums, ref, paths, t, 42)
    print(name, "mode", mode, errs)
    assert errs["ok"] and errs["greek_rel_max"] <= 1e-5, errs  # every Greek within 1e-5 relative


@pytest.mark.parametrize("mode", [1, 2])
def test_ragged_path_count_and_offset(rocm, tapes, mode):
    t = tapes["C2"]
    with rocm.Executable(t, rocm.options("fp64", max_blocks=3, mode=mode)) as x:
        sums, _ = x.replay(513, OFFSET, 0x12345678FEDCBA98)
    ref = oracle.replay_sums(t, 513, OFFSET, 0x12345678FEDCBA98)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-12


def test_run_to_run_bit_identity(rocm, tapes):
    with rocm.Executable(tapes["C2"], rocm.options("fp64")) as x:
        a, _ = x.replay(300_000, 0, 42)
        b, _ = x.replay(300_000, 0, 42)
    assert np.array_equal(a, b)


def test_executables_on_two_threads(rocm, tapes):
    """Two executables, each with its own stream and buffers, created and
    replayed from two threads at once (the library call releases the
    interpreter lock): each thread's sums equal the same replays made one
    after another, bit for bit."""
    import threading

    jobs = {"C2": 200_000, "C3": 100_000}

    def run(name, out):
        with rocm.Executable(tapes[name], rocm.options("fp64")) as x:
            out[name] = [x.replay(jobs[name], k * jobs[name], 42)[0] for k in range(5)]

    print("case two threads C2 and C3", flush=True)
    seq, par = {}, {}
    for name in jobs:
        run(name, seq)
    threads = [threading.Thread(target=run, args=(name, par)) for name in jobs]
    for t in threads:
        t.start()
    for t in threads:
        t.join(timeout=100)
    assert not any(t.is_alive() for t in threads)
    for name in jobs:
        assert name in par, name
        for a, b in zip(seq[name], par[name]):
            assert np.array_equal(a, b), name


def test_dispatch_split_is_additive(rocm, tapes):
    with rocm.Executable(tapes["C2"], rocm.options("fp64")) as x:
        whole, _ = x.replay(100_000, 0, 7)
        first, _ = x.replay(60_000, 0, 7)
        second, _ = x.replay(40_000, 60_000, 7)
    assert rel_err(first + second, whole, floor=1e-300) <= 1e-12


def test_one_dispatch_of_more_than_2_pow_32_paths(rocm, tapes):
    """The European call over 5 x 10^9 paths in one dispatch (a path count
    and path indices past 2^32, about 1,600 paths per lane on the capped grid)
    equals two dispatches of half as many each to 1e-12, and its price is
    Black-Scholes' within four standard errors."""
    from scipy.stats import norm

    n = 5_000_000_000
    print(f"case C1 one dispatch of {n} paths", flush=True)
    with rocm.Executable(tapes["C1"], rocm.options("fp64")) as x:
        whole, _ = x.replay(n, 0, 42)
        first, _ = x.replay(n // 2, 0, 42)
        second, _ = x.replay(n // 2, n // 2, 42)
    assert rel_err(first + second, whole, floor=1e-300) <= 1e-12
    res = oracle.to_result(whole, n)
    s0, k, vol, r, t = 100.0, 100.0, 0.2, 0.03, 1.0
    d1 = (np.log(s0 / k) + (r + 0.5 * vol * vol) * t) / (vol * np.sqrt(t))
    bs = s0 * norm.cdf(d1) - k * np.exp(-r * t) * norm.cdf(d1 - vol * np.sqrt(t))
    assert abs(res["price"] - bs) <= 4 * res["stderr"], (res["price"], bs, res["stderr"])


def test_worst_of_launches_past_2_pow_32_are_additive(rocm, tapes):
    """The worst-of risk run (launch k over scenarios [k 10^6, (k + 1) 10^6))
    reaches counter offsets past 2^32 from launch 4,295 on. Launches 4,294
    (which straddles 2^32) and 4,295 add up to one dispatch over both ranges,
    and 20,000 fp32 paths on either side of 2^32 reconcile with the fp64
    oracle (price and each Greek within 1e-5 relative)."""
    t = tapes["C5"]
    print("case C5 fp32 launches 4294, 4295 and 2^32 - 10^4", flush=True)
    with rocm.Executable(t, rocm.options("fp32")) as x:
        a, _ = x.replay(1_000_000, 4294 * 10**6, 42)
        b, _ = x.replay(1_000_000, 4295 * 10**6, 42)
        ab, _ = x.replay(2_000_000, 4294 * 10**6, 42)
        near, _ = x.replay(20_000, 2**32 - 10_000, 42)
    assert rel_err(a + b, ab, floor=1e-300) <= 1e-12
    ref = oracle.replay_sums(t, 20_000, 2**32 - 10_000, 42)
    r = reconcile(near, ref, 20_000, t, 42, offset=2**32 - 10_000)
    print(r)
    assert r["ok"]


def test_set_inputs_moves_the_market(rocm, tapes):
    t = tapes["C1"]
    with rocm.Executable(t, rocm.options("fp64")) as x:
        x.set_inputs([110.0, 100.0, 0.2, 0.03, 1.0])
        sums, _ = x.replay(50_000, 0, 42)
    ref = oracle.replay_sums(t, 50_000, 0, 42, inputs=[110.0, 100.0, 0.2, 0.03, 1.0])
    assert rel_err(sums, ref, floor=1e-300) <= 1e-10


def test_price_only_kernel(rocm, tapes):
    with rocm.Executable(tapes["C2"], rocm.options("fp64", adjoints=False)) as x:
        sums, _ = x.replay(50_000, 0, 42)
    ref = oracle.replay_sums(tapes["C2"], 50_000, 0, 42, adjoints=False)
    assert abs(sums[0] - ref[0]) <= 1e-10 * abs(ref[0])
    assert np.all(sums[2:] == 0.0)


@pytest.mark.parametrize("name,mode,paths", [("C2", 0, 200_000), ("C4", 0, 20_000), ("C3", 1, 50_000)])
def test_replay_many_equals_separate_replays(rocm, tapes, name, mode, paths):
    """Several input sets in one dispatch (draws shared in tangent mode, one
    replay per set for a reverse-sweep executable): each set's sums equal a
    separate replay with those inputs bit for bit, and the oracle's to 1e-10."""
    t = tapes[name]
    x0 = np.array(t["recorded_inputs"])
    sets = np.stack([x0, x0 * 1.02, x0 * 0.98, x0 * 1.05])
    print(f"case {name} mode={mode} markets=4 paths={paths}", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        many, _ = x.replay_many(sets, paths, OFFSET, 42)
        for m in range(len(sets)):
            x.set_inputs(sets[m])
            one, _ = x.replay(paths, OFFSET, 42)
            assert np.array_equal(many[m], one), m
    ref = oracle.replay_sums(t, paths, OFFSET, 42, inputs=sets[1])
    # price and sum of squares componentwise; the gradient normwise (a Heston
    # gradient component can nearly cancel over 20k paths)
    assert rel_err(many[1][:2], ref[:2], floor=1e-300) <= 1e-10
    assert np.max(np.abs(many[1][2:] - ref[2:])) <= 1e-10 * np.max(np.abs(ref[2:]))


@pytest.mark.parametrize("name,paths", [("C3", 100_000), ("C4", 20_000)])
def test_price_only_replay_many_shares_draws(rocm, tapes, name, paths):
    """A price-only executable runs in the tangent frame with no tangents, so
    several input sets share each path's draws in one dispatch, each set's
    sums equal to a separate price-only replay bit for bit and the price to
    the oracle's to 1e-10."""
    t = tapes[name]
    x0 = np.array(t["recorded_inputs"])
    sets = np.stack([x0 * 0.97, x0, x0 * 1.03])
    print(f"case {name} price only markets=3 paths={paths}", flush=True)
    with rocm.Executable(t, rocm.options("fp64", adjoints=False)) as x:
        assert x.info()["mode"] == 2
        many, _ = x.replay_many(sets, paths, OFFSET, 42)
        for m in range(len(sets)):
            x.set_inputs(sets[m])
            one, _ = x.replay(paths, OFFSET, 42)
            assert np.array_equal(many[m], one), m
            assert np.all(one[2:] == 0.0)
    ref = oracle.replay_sums(t, paths, OFFSET, 42, inputs=sets[2], adjoints=False)
    assert rel_err(many[2][:2], ref[:2], floor=1e-300) <= 1e-10


def test_launch_grid(rocm, tapes):
    """The launch geometry: a long path on the fewest whole blocks per compute
    unit that leave at most two paths per lane, up to 8 resident grids; a
    short path (the European) on at most one resident grid; a reverse sweep
    with its tape in device memory on as many blocks as 1 GiB of tape holds;
    a caller's max_blocks as a hard cap."""
    import ctypes

    hip = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so.7")  # the runtime libnt_rocm.so links
    n = ctypes.c_int(0)
    assert hip.hipDeviceGetAttribute(ctypes.byref(n), 63, 0) == 0  # hipDeviceAttributeMultiprocessorCount
    cus = n.value
    print(f"case launch grid C1 C2, {cus} CUs", flush=True)
    with rocm.Executable(tapes["C2"], rocm.options("fp64")) as x:
        info = x.info()
        assert info["mode"] == 2 and info["tape_slots"] == 0
        resident = info["grid_cap"] // 8
        assert resident % cus == 0
        need = -(-2_000_000 // 256)
        assert x.grid(2_000_000) == (-(-need // (2 * cus)) * cus, 256)
        assert x.grid(2_000_000)[0] * 256 * 2 >= 2_000_000
        assert x.grid(100) == (1, 256)
        assert x.grid(resident * 256)[0] == resident
        assert x.grid(resident * 256 + 1)[0] == resident
        assert x.grid(10**12)[0] == info["grid_cap"]
        with pytest.raises(rocm.NtError):
            x.grid(0)
    with rocm.Executable(tapes["C2"], rocm.options("fp64", max_blocks=100)) as x:
        assert x.info()["grid_cap"] == 100 and x.grid(2_000_000)[0] == 100 and x.grid(1000)[0] == 4
    with rocm.Executable(tapes["C2"], rocm.options("fp64", mode=1, checkpoint=2)) as x:
        info = x.info()
        assert info["tape_slots"] > 0 and x.grid(2_000_000)[0] == info["grid_cap"]
        assert info["grid_cap"] * 256 * info["tape_slots"] * 8 <= 1 << 30 and info["grid_cap"] % cus == 0
    with rocm.Executable(tapes["C1"], rocm.options("fp64")) as x:
        info = x.info()
        assert x.grid(1_000_000)[0] <= info["grid_cap"] and x.grid(10**9)[0] == info["grid_cap"]


@pytest.mark.parametrize("mode", [2, 1])
def test_sums_do_not_depend_on_the_grid(rocm, tapes, mode):
    """The launch grid decides only which lane takes which path and the order
    of the partial sums: the default grid (more blocks than the device holds)
    and a grid capped at 256 blocks give the same sums to rounding, and the
    same per-path values bit for bit."""
    t = tapes["C2"]
    paths = 1_000_000
    print(f"case C2 mode={mode} grid independence, {paths} paths", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        g = x.grid(paths)[0]
        assert g * 256 < paths  # more than one path per lane, more blocks than 256
        a, _ = x.replay(paths, OFFSET, 42)
        va, ga = x.replay_paths(2_000, OFFSET, 42)
    with rocm.Executable(t, rocm.options("fp64", mode=mode, max_blocks=256)) as x:
        assert x.grid(paths)[0] == 256 != g
        b, _ = x.replay(paths, OFFSET, 42)
        vb, gb = x.replay_paths(2_000, OFFSET, 42)
    assert rel_err(a, b, floor=1e-300) <= 1e-12
    assert np.array_equal(va, vb) and np.array_equal(ga, gb)


@pytest.mark.parametrize("name", ["C2", "C4"])
def test_replay_many_with_a_non_finite_set(rocm, tapes, name):
    """One input set of several with a NaN first input: its lanes go to the
    exception kernel for that set alone, its sums have the oracle's NaN
    pattern, and the other sets' sums equal separate replays bit for bit."""
    t = tapes[name]
    x0 = np.array(t["recorded_inputs"])
    bad = x0.copy()
    bad[0] = np.nan
    sets = np.stack([x0, bad, x0 * 1.01])
    paths = 20_000
    print(f"case {name} replay_many with a NaN set", flush=True)
    with rocm.Executable(t, rocm.options("fp64")) as x:
        many, _ = x.replay_many(sets, paths, OFFSET, 42)
        for m in (0, 2):
            x.set_inputs(sets[m])
            one, _ = x.replay(paths, OFFSET, 42)
            assert np.array_equal(many[m], one), m
    want = oracle.replay_sums(t, paths, OFFSET, 42, inputs=bad)
    assert np.array_equal(np.isnan(many[1]), np.isnan(want)), (many[1], want)


def test_dispatch_timing_is_ordered(rocm, tapes):
    """The three timing figures of a dispatch: the replay kernel (first two
    events), all its kernels (first to last event) and the host's wall time,
    in that order and positive; the same for a dispatch of several sets."""
    t = tapes["C2"]
    print("case timing C2 and C1", flush=True)
    for name, paths in (("C2", 2_000_000), ("C1", 1_000_000)):
        with rocm.Executable(tapes[name], rocm.options("fp64")) as x:
            for _ in range(3):
                _, tm = x.replay(paths, 0, 42)
                assert 0.0 < tm["replay_ms"] <= tm["kernel_ms"] <= tm["wall_ms"], (name, tm)
    with rocm.Executable(t, rocm.options("fp64")) as x:
        x0 = np.array(t["recorded_inputs"])
        _, tm = x.replay_many(np.stack([x0, x0 * 1.01]), 200_000, 0, 42)
        assert 0.0 < tm["kernel_ms"] <= tm["wall_ms"], tm


@pytest.mark.parametrize("mode", [2, 1])
def test_degenerate_tapes(rocm, nt, mode):
    """No draws, an output that is an input, a zero derivative, an output that
    is a draw: per path and summed against the oracle."""
    for name, flat in degenerate_tapes(nt).items():
        print(f"case degenerate tape {name} mode {mode}", flush=True)
        with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
            sums, _ = x.replay(100_000, OFFSET, 42)
            assert rel_err(sums, oracle.replay_sums(flat, 100_000, OFFSET, 42), floor=1e-300) <= 1e-10, name
            v, g = x.replay_paths(1000, OFFSET, 42)
            ov, og = oracle.replay_paths(flat, 1000, OFFSET, 42)
            assert rel_err(v, ov) <= 1e-12 and rel_err(g, og) <= 1e-12, name


@pytest.mark.parametrize("precision,mode", [("fp64", 2), ("fp64", 1), ("fp32", 2)])
def test_tape_with_no_inputs(rocm, nt, precision, mode):
    """A price with no inputs: two sums (Σy, Σy²) and no derivative columns,
    against the oracle (fp32 against the fp64 oracle at 1e-5)."""
    flat = no_input_tape(nt).flat()
    print(f"case no-input tape {precision} mode {mode}", flush=True)
    with rocm.Executable(flat, rocm.options(precision, mode=mode)) as x:
        x.set_inputs([])
        sums, _ = x.replay(200_000, OFFSET, 42)
        want = oracle.replay_sums(flat, 200_000, OFFSET, 42)
        assert len(sums) == 2
        assert rel_err(sums, want, floor=1e-300) <= (1e-10 if precision == "fp64" else 1e-5)
        if precision == "fp64":
            v, g = x.replay_paths(4096, OFFSET, 42)
            ov, _ = oracle.replay_paths(flat, 4096, OFFSET, 42)
            assert g.shape == (4096, 0)
            assert rel_err(v, ov) <= 1e-12


@pytest.mark.parametrize("mode", [2, 1])
def test_tiny_counts_and_an_offset_that_wraps(rocm, tapes, mode):
    """Dispatches of 1 to 257 paths (one partly filled block, a partial wave)
    and a range of paths whose 64-bit index wraps past 2^64 - 1: sums against
    the oracle's over the same paths to 1e-10, per path within the bar."""
    t = tapes["C2"]
    print(f"case C2 mode={mode} tiny counts and a wrapping offset", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        for paths, offset in [(1, 0), (2, OFFSET), (63, 5), (64, 0), (65, OFFSET), (255, 1), (257, 77),
                              (16, 2**64 - 7)]:
            got, _ = x.replay(paths, offset, 42)
            want = oracle.replay_sums(t, paths, offset, 42)
            assert rel_err(got, want, floor=1e-300) <= 1e-10, (paths, offset)
        v, g = x.replay_paths(16, 2**64 - 7, 42)
    check_per_path(v, g, t, 16, 2**64 - 7, 42, min_strict=0.8, max_above=0.25)


@pytest.mark.parametrize("name,precision", [("C2", "fp64"), ("C3", "fp32")])
def test_replay_many_beyond_one_kernel(rocm, tapes, name, precision):
    """Thirteen input sets: more than one multi-market kernel holds at two
    waves per SIMD, so the dispatch is split into kernels of a few sets each;
    every set's sums still equal a separate replay bit for bit."""
    t = tapes[name]
    x0 = np.array(t["recorded_inputs"])
    sets = np.stack([x0 * (1.0 + 0.004 * (m - 6)) for m in range(13)])
    paths = 50_000
    print(f"case {name} {precision} replay_many of 13 sets", flush=True)
    with rocm.Executable(t, rocm.options(precision)) as x:
        many, _ = x.replay_many(sets, paths, OFFSET, 42)
        for m in range(len(sets)):
            x.set_inputs(sets[m])
            one, _ = x.replay(paths, OFFSET, 42)
            assert np.array_equal(many[m], one), m


def test_replay_many_of_one_set_and_bad_arguments(rocm, tapes):
    t = tapes["C2"]
    with rocm.Executable(t, rocm.options("fp64")) as x:
        one, _ = x.replay(10_000, 0, 7)
        many, _ = x.replay_many(np.array([t["recorded_inputs"]]), 10_000, 0, 7)
        assert np.array_equal(many[0], one)
        with pytest.raises(ValueError):
            x.replay_many(np.zeros((2, 3)), 10_000, 0, 7)


@pytest.mark.parametrize("mode", [1, 2])
def test_uniforms_and_named_streams_per_path(rocm, nt, mode):
    """The reference's random-streams body rolled over 64 steps: per path
    against the oracle (reverse sweep and tangent mode)."""
    from conftest import jump_clock_tape
    flat = jump_clock_tape(nt, 64).flat()
    print(f"case jump-clock mode={mode}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
        v, g = x.replay_paths(2048, OFFSET, 42)
        sums, _ = x.replay(200_000, 0, 42)
    print(check_per_path(v, g, flat, 2048, OFFSET, 42))
    ref = oracle.replay_sums(flat, 200_000, 0, 42)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-10


@pytest.mark.parametrize("seed", [301, 302, 303])
def test_random_tapes_every_operation_on_device(rocm, nt, seed):
    """Straight-line tapes of random shape using every operation, normals on
    two streams and uniforms (conftest.random_tape), one output: per path and
    summed against the oracle in both sweeps. At 250 steps (over 512 nodes)
    the reverse sweep cuts the tape into checkpointed segments."""
    from conftest import random_tape
    for steps in (120, 250):
        flat = random_tape(nt, seed, steps, outputs=1).flat()
        for mode in (2, 1):
            print(f"case random tape seed={seed} steps={steps} mode={mode}", flush=True)
            with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
                info = x.info()
                assert info["scratch_bytes"] == 0 and info["mode"] == mode
                assert (info["n_segments"] > 0) == (mode == 1 and steps == 250)
                v, g = x.replay_paths(1024, OFFSET, 42)
                sums, _ = x.replay(100_000, 0, 42)
            check_per_path(v, g, flat, 1024, OFFSET, 42, max_above=0.0)
            assert rel_err(sums, oracle.replay_sums(flat, 100_000, 0, 42), floor=1e-300) <= 1e-10


@pytest.mark.parametrize("builder", ["jump_clock_tape", "two_output_tape"])
def test_uniforms_streams_and_outputs_fp32_reconcile(rocm, nt, builder):
    """The uniform and named-stream tape and the two-output tape in fp32
    against the fp64 oracle: the price and every Greek within 1e-5 relative,
    but for the terminal spot's vega, which is zero in expectation (E[S_T] =
    S0 e^{rT} whatever the volatility), so that its Monte-Carlo mean is noise
    (-0.30 against a rho of 103) and it is held with the other Greeks of its
    output within 1e-5 normwise (max_j |dg_j| / max_j |g_j|)."""
    import conftest
    flat = getattr(conftest, builder)(nt).flat()
    paths = 200_000
    print(f"case {builder} fp32 paths={paths}", flush=True)
    with rocm.Executable(flat, rocm.options("fp32")) as x:
        sums, _ = x.replay(paths, 0, 42)
    ref = oracle.replay_sums(flat, paths, 0, 42, all_outputs=True)
    row = 2 + len(flat["input_node"])
    for o in range(len(flat["output_node"])):
        r = reconcile(sums[o * row:(o + 1) * row], ref[o * row:(o + 1) * row], paths, flat, 42)
        print(o, r)
        if builder == "two_output_tape" and o == 0:
            assert r["price"] <= 1e-5 and r["normwise"] <= 1e-5, r
            got = oracle.to_result(sums[:row], paths)["gradient"]
            want = oracle.to_result(ref[:row], paths)["gradient"]
            for j in (0, 2):  # delta and rho
                assert abs(got[j] - want[j]) <= 1e-5 * abs(want[j]), (j, got[j], want[j])
        else:
            assert r["ok"], o


def test_multi_output_per_path_and_sums(rocm, nt):
    from conftest import two_output_tape
    flat = two_output_tape(nt).flat()
    print("case two outputs", flush=True)
    with rocm.Executable(flat, rocm.options("fp64")) as x:
        assert x.info()["mode"] == 2
        v, g = x.replay_paths(2048, OFFSET, 42)
        sums, _ = x.replay(200_000, 0, 42)
        many, _ = x.replay_many(np.stack([flat["recorded_inputs"], np.array(flat["recorded_inputs"]) * 1.1]),
                                200_000, 0, 42)
    assert v.shape == (2048, 2) and g.shape == (2048, 2, 3)
    ov, og = oracle.replay_paths(flat, 2048, OFFSET, 42, output=None)
    for o in range(2):
        ev, eg = oracle.path_errors(v[:, o], g[:, o, :], ov[:, o], og[:, o, :])
        assert ev.max() <= 1e-12 and eg.max() <= 1e-12, o
    ref = oracle.replay_sums(flat, 200_000, 0, 42, all_outputs=True)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-10
    assert np.array_equal(many[0], sums)


@pytest.mark.parametrize("a,tol", [(0.3, 1e-12), (110.0, 1e-10)])
def test_loop_exponent_bound_on_device(rocm, nt, a, tol):
    """s exp(a z) over 16 steps, tangent mode: the exponents are bounded once
    per path before the loop. With a = 0.3 every path stays on the table exp;
    with a = 110 the bound (6.77 |a| = 745 > 708) sends every path to the
    device-libm evaluation. The exponent a z multiplies the normals' own
    difference from the oracle's (a few 1e-15) by a at each step, so a = 110
    is held to 1e-10 per path."""
    from conftest import scaled_exp_tape
    flat = scaled_exp_tape(nt, a).flat()
    print(f"case scaled exp a={a}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=2)) as x:
        assert x.info()["mode"] == 2
        v, g = x.replay_paths(4096, OFFSET, 5)
    ov, og = oracle.replay_paths(flat, 4096, OFFSET, 5)
    ev, eg = oracle.path_errors(v, g, ov, og)
    finite = np.isfinite(ov) & np.isfinite(og).all(axis=1) & (np.abs(og) < 1e300).all(axis=1)
    assert finite.sum() > 3000
    assert ev.max() <= tol and eg[finite].max() <= tol, (ev.max(), eg[finite].max())


@pytest.mark.parametrize("s_val,floor", [(1e-3, True), (1e-310, True), (1e-3, False)])
def test_sqrt_routine_and_fallback_on_device(rocm, nt, s_val, floor):
    """SQRT nodes in a tangent kernel: +0 arguments stay on nt_sqrt_q,
    subnormal (s = 1e-310) and negative (no floor) arguments send the path to
    device-libm sqrt; values and derivatives per path against the oracle,
    NaN for NaN."""
    from conftest import sqrt_classes_tape
    flat = sqrt_classes_tape(nt, s_val, floor).flat()
    print(f"case sqrt classes s={s_val} floor={floor}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=2)) as x:
        v, g = x.replay_paths(4096, OFFSET, 9)
    ov, og = oracle.replay_paths(flat, 4096, OFFSET, 9)
    ev, eg = oracle.path_errors(v, g, ov, og)
    assert ev.max() <= 1e-12 and eg.max() <= 1e-12, (ev.max(), eg.max())
    assert np.array_equal(np.isnan(v), np.isnan(ov))


@pytest.mark.parametrize("precision,mode", [("fp64", 2), ("fp64", 1), ("fp32", 2)])
def test_max_min_follow_java_math_on_device(rocm, nt, precision, mode):
    """MAX and MIN per path against the oracle's java.lang.Math.max/min on
    signed zeros, NaN and infinities (two inputs, and an input and a literal):
    the value with its sign of zero, NaN where the oracle has NaN."""
    from conftest import MAX_MIN_CASES, MAX_MIN_OUTPUTS, max_min_tape, same_special
    tapes_ = [max_min_tape(nt).flat()] if mode == 2 else [max_min_tape(nt, o).flat() for o in range(MAX_MIN_OUTPUTS)]
    print(f"case MAX/MIN edge cases {precision} mode={mode}", flush=True)
    for flat in tapes_:
        with rocm.Executable(flat, rocm.options(precision, mode=mode)) as x:
            for case in MAX_MIN_CASES:
                x.set_inputs(list(case))
                v, _ = x.replay_paths(64, 0, 42)
                ov, _ = oracle.replay_paths(flat, 64, 0, 42, inputs=list(case), f32=precision == "fp32", output=None)
                assert same_special(np.reshape(v, ov.shape), ov), (case, v[:1], ov[:1])


@pytest.mark.parametrize("precision,mode,rel", [("fp64", 2, 5e-16), ("fp64", 1, 5e-16), ("fp32", 2, 4e-7)])
def test_special_values_follow_the_oracle_on_device(rocm, nt, precision, mode, rel):
    """EXP, LOG, SQRT, DIV, 1 / x, ABS, NEG and MUL at signed zeros,
    subnormals, infinities, NaN and the exponential's overflow and underflow,
    per path against the oracle (fp32: the fp32 oracle): the same NaNs,
    infinities and signed zeros, finite values within `rel`."""
    from conftest import SPECIAL_CASES, SPECIAL_OUTPUTS, close_special, special_ops_tape
    tapes_ = [special_ops_tape(nt).flat()] if mode == 2 else [special_ops_tape(nt, o).flat() for o in range(SPECIAL_OUTPUTS)]
    print(f"case special values {precision} mode={mode}", flush=True)
    for flat in tapes_:
        with rocm.Executable(flat, rocm.options(precision, mode=mode)) as x:
            for case in SPECIAL_CASES:
                x.set_inputs(list(case))
                v, g = x.replay_paths(64, 0, 42)
                ov, og = oracle.replay_paths(flat, 64, 0, 42, inputs=list(case), f32=precision == "fp32", output=None)
                assert close_special(np.reshape(v, ov.shape), ov, rel), (case, flat["output_node"], v[:1], ov[:1])
                if mode == 1:  # the reverse sweep's adjoints too
                    assert close_special(np.reshape(g, og.shape), og, rel), (case, flat["output_node"], g[:1], og[:1])


@pytest.mark.parametrize("mode", [2, 1])
def test_non_finite_inputs_give_non_finite_sums_and_leave_the_executable_usable(rocm, tapes, mode):
    """A NaN spot or an infinite volatility sends every lane to the exception
    kernel, whose device-libm replay returns the non-finite sums the oracle
    returns (NaN where it has NaN); the executable then replays finite inputs
    exactly as before."""
    t = tapes["C2"]
    x0 = list(t["recorded_inputs"])
    paths = 20_000
    print(f"case C2 mode={mode} non-finite inputs", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        before, _ = x.replay(paths, OFFSET, 42)
        for bad in ([float("nan"), *x0[1:]], [*x0[:2], float("inf"), *x0[3:]]):
            x.set_inputs(bad)
            got, _ = x.replay(paths, OFFSET, 42)
            want = oracle.replay_sums(t, paths, OFFSET, 42, inputs=bad)
            assert not np.all(np.isfinite(got)), got
            assert np.array_equal(np.isnan(got), np.isnan(want)), (got, want)
            assert np.array_equal(np.isposinf(got), np.isposinf(want)) and np.array_equal(np.isneginf(got), np.isneginf(want))
        x.set_inputs(x0)
        after, _ = x.replay(paths, OFFSET, 42)
    assert np.array_equal(before, after)


@pytest.mark.parametrize("basis", [1, 2])
@pytest.mark.parametrize("name,paths", [("C2", 2048), ("C3", 1024), ("C4", 512), ("C5", 256)])
def test_loop_tangents_over_inputs_and_parameters_on_device(rocm, tapes, name, paths, basis):
    """The step loop's tangents forced over the inputs (basis 1) and over the
    loop's parameters (basis 2): per path within the bar of the oracle."""
    t = tapes[name]
    print(f"case {name} basis={basis} paths={paths}", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=2, basis=basis)) as x:
        v, g = x.replay_paths(paths, OFFSET, 42)
        info = x.info()
    assert info["scratch_bytes"] == 0
    print(check_per_path(v, g, t, paths, OFFSET, 42, min_strict=STRICT[name], max_above=ABOVE[name]))


def test_worst_of_fp32_over_parameters_reconciles(rocm, tapes):
    """The fp32 worst-of kernel (tangents over the loop's parameters) against
    the fp64 oracle over 20,000 paths: price and each of the 33 Greeks within
    1e-5 relative, and 1e-5 normwise (conftest.reconcile)."""
    t = tapes["C5"]
    print("case C5 fp32 paths=20000", flush=True)
    src = rocm.lower(t, rocm.options("fp32", mode=2))
    assert "basis=params" in src
    with rocm.Executable(t, rocm.options("fp32", mode=2)) as x:
        sums, _ = x.replay(20_000, 0, 42)
    errs = reconcile(sums, oracle.replay_sums(t, 20_000, 0, 42), 20_000, t, 42)
    print(errs)
    assert errs["ok"], errs


MERTON = dict(spot=100.0, strike=100.0, vol=0.18, rate=0.03, maturity=1.0, jumpIntensity=0.75, jumpMean=-0.05,
              jumpVol=0.15)


@pytest.mark.parametrize("mode", [1, 2])
def test_merton_jump_tape_per_path(rocm, nt, mode):
    """The Merton jump-diffusion call (MertonJumpModel.european, 128 steps: a
    normal, a uniform and a normal per step) per path against the oracle."""
    from conftest import merton_call_tape
    flat = merton_call_tape(nt, MERTON).flat()
    print(f"case merton mode={mode} paths=2048", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
        v, g = x.replay_paths(2048, OFFSET, 42)
        assert x.info()["loop_period"] > 0
    print(check_per_path(v, g, flat, 2048, OFFSET, 42, min_strict=0.94))  # measured 0.947


def test_merton_jump_tape_several_markets(rocm, nt):
    """The Merton tape priced for three input sets in one dispatch: its lanes
    leave paths to the exception kernel in every market, each market with its
    own lane bitmap, and each market's sums equal a separate replay's bit for
    bit; a second, smaller dispatch of the three sets (on a smaller grid)
    again equals a separate replay, so the first left its bitmaps clear, and
    the oracle's sums within 1e-10."""
    from conftest import merton_call_tape
    flat = merton_call_tape(nt, MERTON, steps=32).flat()
    x0 = np.array(flat["recorded_inputs"])
    sets = np.stack([x0, x0 * 1.03, x0 * 0.97])
    paths = 100_000
    print(f"case merton32 markets=3 paths={paths}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64")) as x:
        assert "nt_replay_slow" in x.source()
        many, _ = x.replay_many(sets, paths, OFFSET, 42)
        for m in range(len(sets)):
            x.set_inputs(sets[m])
            one, _ = x.replay(paths, OFFSET, 42)
            assert np.all(np.isfinite(one)) and np.array_equal(many[m], one), m
        many2, _ = x.replay_many(sets, 20_000, OFFSET, 42)
        x.set_inputs(sets[2])
        one, _ = x.replay(20_000, OFFSET, 42)
        assert np.array_equal(many2[2], one)
    ref = oracle.replay_sums(flat, 20_000, OFFSET, 42, inputs=sets[2])
    assert rel_err(one, ref, floor=1e-300) <= 1e-10


@pytest.mark.parametrize("mode", [2, 1])
def test_exception_kernel_on_grids_off_the_xcd_multiple(rocm, nt, mode):
    """The Merton tape, whose lanes leave paths to the exception kernel, on
    grids of 1, 3, 12 and 14 blocks, and capped at 13 blocks over 100,000
    paths: each channel's column groups the blocks by block mod 8 and puts
    the exception kernel's entries in a second region, and the sums stay the
    oracle's on grids that are not a multiple of 8."""
    from conftest import merton_call_tape
    flat = merton_call_tape(nt, MERTON, steps=32).flat()
    with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
        assert "nt_replay_slow" in x.source()
        for paths, blocks in ((1, 1), (700, 3), (3000, 12), (3329, 14)):
            print(f"case merton32 mode={mode} paths={paths}", flush=True)
            assert x.grid(paths)[0] == blocks
            got, _ = x.replay(paths, OFFSET, 42)
            assert rel_err(got, oracle.replay_sums(flat, paths, OFFSET, 42)) <= 1e-10, paths
    print(f"case merton32 mode={mode} paths=100000 max_blocks=13", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=mode, max_blocks=13)) as x:
        assert x.grid(100_000)[0] == 13
        got, _ = x.replay(100_000, OFFSET, 42)
        assert rel_err(got, oracle.replay_sums(flat, 100_000, OFFSET, 42)) <= 1e-10


def test_merton_jump_tape_converges_to_the_poisson_series(rocm, nt):
    """JumpModelsTest.mertonMonteCarloConvergesToThePoissonSeries at its own
    size (1,500,000 scenarios, seed 42, 128 steps): the device sums agree with
    the oracle's within 1e-10 and the price is within 1.5% of the exact
    Poisson-series price (docs/examples/jump-models.md:48-50)."""
    from conftest import merton_call_tape, merton_series_call
    flat = merton_call_tape(nt, MERTON).flat()
    paths = 1_500_000
    print(f"case merton series paths={paths}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64")) as x:
        sums, _ = x.replay(paths, 0, 42)
    ref = oracle.replay_sums(flat, paths, 0, 42)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-10
    price = oracle.to_result(sums, paths)["price"]
    exact = merton_series_call(100, 100, 1.0, 0.03, 0.18, 0.75, -0.05, 0.15)
    print(f"price {price:.6f} series {exact:.6f} rel {(price - exact) / exact:.2e}")
    assert abs(price - exact) <= 0.015 * exact


@pytest.mark.parametrize("mode", [1, 2])
def test_step_schedule_recorded_up_front_on_device(rocm, mode):
    """The Asian call on TimeGrid.of 252 weekday fixings (its per-step drift
    and diffusion recorded before the first step, GbmPath.java:61-66) runs as
    a rolled loop with a per-step fraction table: no scratch, per path within
    the bar, sums within 1e-10 of the oracle's."""
    from nablatensor_amd import workloads
    flat = workloads.schedule_tapes()["asian_weekdays"].flat()
    print(f"case asian_weekdays mode={mode}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
        info = x.info()
        assert info["scratch_bytes"] == 0 and info["loop_period"] == 11
        v, g = x.replay_paths(2048, OFFSET, 42)
        sums, _ = x.replay(200_000, 0, 42)
    print(check_per_path(v, g, flat, 2048, OFFSET, 42, min_strict=0.94))  # measured 0.943
    ref = oracle.replay_sums(flat, 200_000, 0, 42)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-10


def test_step_schedule_per_block_fp32_and_a_tail_trip(rocm, nt):
    """The weekday Asian's tangent kernels with the step schedule computed once
    per block: fp32 reconciles with the fp64 oracle (price and each Greek within
    1e-5 relative); a 64-fixing grid (a lead step
    and 31 trips of two) and a 400-fixing grid (399 loop steps, more than a
    block's 256 threads, so threads stride over the schedule's steps; a lead
    step, 199 trips and a tail of one) are per path within the bar in fp64."""
    from nablatensor_amd import workloads
    flat = workloads.schedule_tapes()["asian_weekdays"].flat()
    print("case asian_weekdays fp32 tangent, 20000 paths", flush=True)
    with rocm.Executable(flat, rocm.options("fp32", mode=2)) as x:
        sums, _ = x.replay(20_000, 0, 42)
    errs = reconcile(sums, oracle.replay_sums(flat, 20_000, 0, 42), 20_000, flat, 42)
    print(errs)
    assert errs["ok"], errs
    for fixings in (64, 400):
        grid = nt.TimeGrid.of(workloads.weekday_fixings(fixings))
        flat = nt.record(nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), grid).flat()
        print(f"case weekday {fixings} fixings fp64 tangent, 1000 paths", flush=True)
        with rocm.Executable(flat, rocm.options("fp64", mode=2)) as x:
            src = x.source()
            assert "it0 = 1u + (sg) * 2u" in src and "schedule=0" not in src
            v, g = x.replay_paths(1000, OFFSET, 42)
            sums, _ = x.replay(1000, OFFSET, 42)
        print(check_per_path(v, g, flat, 1000, OFFSET, 42, min_strict=0.9))
        assert rel_err(sums, oracle.replay_sums(flat, 1000, OFFSET, 42), floor=1e-300) <= 1e-10


def test_discounted_weekday_asian_growth_from_the_schedule(rocm, nt):
    """A bank account b <- b * exp(r * dt_i) on a 48-fixing weekday grid: the
    growth factor is path-invariant, so the tangent kernel reads it (and its
    rate tangent) from the per-block schedule. Per path within the bar, sums
    within 1e-10 (the rate sensitivity nearly cancels, so floored at 1)."""
    from conftest import discounted_weekday_asian_tape
    flat = discounted_weekday_asian_tape(nt, 48)
    print("case discounted weekday asian, 48 fixings fp64 tangent, 1000 paths", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=2)) as x:
        assert "schedule=0" not in x.source()
        v, g = x.replay_paths(1000, OFFSET, 42)
        sums, _ = x.replay(1000, OFFSET, 42)
    print(check_per_path(v, g, flat, 1000, OFFSET, 42, min_strict=0.85))
    assert rel_err(sums, oracle.replay_sums(flat, 1000, OFFSET, 42), floor=1.0) <= 1e-10


def test_signed_affine_exponents_on_device(rocm, nt):
    """Spots whose step exponents are p - r w (w a correlated normal), r z - p
    and r z, summed as their draws and formed after the loop: per path within
    the bar (fp64), sums within 1e-10 of the oracle's; fp32 (exponents folded
    into exp2) reconciles with the fp64 oracle."""
    from conftest import signed_basket_tape
    flat = signed_basket_tape(nt, 40)
    print("case signed basket, 40 steps fp64 tangent, 2048 paths", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=2)) as x:
        assert x.source().count("real zq0_") >= 3
        v, g = x.replay_paths(2048, OFFSET, 42)
        sums, _ = x.replay(2048, OFFSET, 42)
    print(check_per_path(v, g, flat, 2048, OFFSET, 42, min_strict=0.9))
    ref = oracle.replay_sums(flat, 20_000, OFFSET, 42)
    assert rel_err(sums, oracle.replay_sums(flat, 2048, OFFSET, 42), floor=1.0) <= 1e-10
    print("case signed basket, 40 steps fp32 tangent, 20000 paths", flush=True)
    with rocm.Executable(flat, rocm.options("fp32", mode=2)) as x:
        assert x.source().count("real zq0_") >= 3
        sums, _ = x.replay(20_000, OFFSET, 42)
    errs = reconcile(sums, ref, 20_000, flat, 42, offset=OFFSET)
    print(errs)
    assert errs["ok"], errs


def _line_tape(nt, tapes, name):
    from conftest import branching_tape
    from nablatensor_amd import workloads
    if name == "weekdays":
        return workloads.schedule_tapes()["asian_weekdays"].flat()
    if name == "branching":
        return branching_tape(nt).flat()
    return tapes[name]


@pytest.mark.parametrize("name,libm,seg,paths,strict", [
    ("C2", 0, 0, 2048, STRICT["C2"]), ("C2", 1, 0, 2048, STRICT["C2"]), ("C3", 0, 0, 1024, STRICT["C3"]),
    ("weekdays", 0, 0, 2048, 0.94), ("branching", 0, 19, 4096, 1.0)])
def test_checkpointed_straight_line_on_device(rocm, nt, tapes, name, libm, seg, paths, strict):
    """Tapes lowered without a step loop and swept in reverse segment by
    segment (the reference's segment-checkpoint plan, AadCheckpointPlan.java:95-172):
    no scratch, per path within the bar, sums within 1e-10 of the oracle's.
    With device libm Box-Muller the 252-fixing Asian is within 1e-12 on every
    path."""
    flat = _line_tape(nt, tapes, name)
    print(f"case straight line {name} libm={libm} seg={seg} paths={paths}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", roll=-1, mode=1, libm=libm, seg_len=seg)) as x:
        info = x.info()
        assert info["scratch_bytes"] == 0 and info["loop_period"] == 0
        assert info["n_segments"] > 1 and info["checkpoint"] == rocm.NT_CKPT_RECOMPUTE
        v, g = x.replay_paths(paths, OFFSET, 42)
        sums, _ = x.replay(100_000, 0, 42)
    print(info["vgprs"], "VGPRs", info["n_segments"], "segments", info["tape_slots"], "stored")
    out = check_per_path(v, g, flat, paths, OFFSET, 42, min_strict=strict)
    print(out)
    if libm:
        assert out["max_err"] <= 1e-12, out
    ref = oracle.replay_sums(flat, 100_000, 0, 42)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-10


def test_checkpointed_straight_line_exception_kernel_on_device(rocm, nt):
    """The 32-step Merton jump tape without its loop, in 40-node segments:
    the paths whose indicator overflows exp go to the exception kernel, which
    re-evaluates them segment by segment; per path within the bar."""
    from conftest import merton_call_tape
    flat = merton_call_tape(nt, MERTON, steps=32).flat()
    print("case straight line merton seg=40 paths=2048", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", roll=-1, mode=1, seg_len=40)) as x:
        assert x.info()["n_segments"] > 1
        v, g = x.replay_paths(2048, OFFSET, 42)
    assert np.all(np.isfinite(g))
    print(check_per_path(v, g, flat, 2048, OFFSET, 42, min_strict=0.98))  # measured 0.985


def test_checkpointed_straight_line_fp32_reconciles(rocm, tapes):
    """fp32, the 252-fixing Asian without its loop, reverse sweep in segments:
    price and each Greek within 1e-5 relative of the fp64 oracle."""
    t = tapes["C2"]
    paths = 200_000
    print(f"case straight line C2 fp32 paths={paths}", flush=True)
    with rocm.Executable(t, rocm.options("fp32", roll=-1, mode=1)) as x:
        assert x.info()["n_segments"] > 1 and x.info()["scratch_bytes"] == 0
        sums, _ = x.replay(paths, 0, 42)
    ref = oracle.replay_sums(t, paths, 0, 42)
    r = reconcile(sums, ref, paths, t, 42)
    print(r)
    assert r["ok"]


@pytest.mark.parametrize("mode", [0, 1, 2])
def test_local_vol_tape_per_path(rocm, mode):
    """The Asian under a parametric local volatility with 24 coefficients (27
    inputs; workloads.local_vol_asian_tape), where the reverse sweep runs 1.5x
    faster than tangent mode: the cost model picks the reverse sweep (mode
    0), and both sweeps match the oracle per path within the bar, with no
    scratch."""
    from nablatensor_amd import workloads
    flat = workloads.local_vol_asian_tape(24).flat()
    print(f"case local_vol k=24 mode={mode} paths=512", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
        info = x.info()
        assert info["scratch_bytes"] == 0
        assert info["mode"] == (1 if mode == 0 else mode)
        v, g = x.replay_paths(512, OFFSET, 42)
    print(check_per_path(v, g, flat, 512, OFFSET, 42, min_strict=0.88))  # measured 0.891
