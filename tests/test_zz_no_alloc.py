"""The allocation-free entry point nt_exec_replay_noalloc against nt_exec_replay.

nt_exec_replay_noalloc runs the same replay and finishing kernels with the
per-block partials (and a reverse sweep's per-lane tape) in the library's
static device array, reading inputs from and writing sums to device memory
the caller passes. Its sums must be bit-identical to nt_exec_replay's for the
same inputs, paths, offset and seed, on consecutive calls (the second smaller,
so stale partials of the first would show), and a dispatch whose scratch
would not fit must be refused before anything runs.
"""
from __future__ import annotations

import ctypes as C

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

OFFSET = 0x100000003


class Hip:
    """The few HIP runtime calls the test needs to own device buffers, from the
    same libamdhip64 that libnt_rocm.so links."""

    def __init__(self):
        self.L = C.CDLL("/opt/rocm/lib/libamdhip64.so.7")
        self.L.hipMalloc.argtypes = [C.POINTER(C.c_void_p), C.c_size_t]
        self.L.hipFree.argtypes = [C.c_void_p]
        self.L.hipMemcpy.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t, C.c_int]
        self.L.hipStreamCreate.argtypes = [C.POINTER(C.c_void_p)]
        self.L.hipStreamSynchronize.argtypes = [C.c_void_p]
        self.L.hipStreamDestroy.argtypes = [C.c_void_p]
        self.L.hipMemset.argtypes = [C.c_void_p, C.c_int, C.c_size_t]
        self.L.hipStreamBeginCapture.argtypes = [C.c_void_p, C.c_int]
        self.L.hipStreamEndCapture.argtypes = [C.c_void_p, C.POINTER(C.c_void_p)]
        self.L.hipGraphInstantiate.argtypes = [C.POINTER(C.c_void_p), C.c_void_p, C.c_void_p, C.c_char_p, C.c_size_t]
        self.L.hipGraphLaunch.argtypes = [C.c_void_p, C.c_void_p]
        self.L.hipGraphExecDestroy.argtypes = [C.c_void_p]
        self.L.hipGraphDestroy.argtypes = [C.c_void_p]

    def ok(self, rc):
        assert rc == 0, f"HIP error {rc}"

    def malloc(self, nbytes):
        p = C.c_void_p()
        self.ok(self.L.hipMalloc(C.byref(p), nbytes))
        return p

    def to_device(self, arr):
        a = np.ascontiguousarray(arr, dtype=np.float64)
        p = self.malloc(max(8, a.nbytes))
        self.ok(self.L.hipMemcpy(p, a.ctypes.data, a.nbytes, 1))  # hipMemcpyHostToDevice
        return p

    def to_host(self, p, n):
        out = np.zeros(n, dtype=np.float64)
        self.ok(self.L.hipMemcpy(out.ctypes.data, p, out.nbytes, 2))  # hipMemcpyDeviceToHost
        return out


@pytest.fixture(scope="module")
def rocm():
    from nablatensor_amd import rocm as r
    assert r.probe() > 0, "no gfx950 device visible to libnt_rocm.so"
    return r


@pytest.fixture(scope="module")
def hip(rocm):
    return Hip()


def noalloc(rocm, hip, x, inputs, paths, offset, seed, stream=None):
    L = rocm.lib()
    n_sums = x.n_outputs * (2 + x.n_inputs)
    d_in = hip.to_device(inputs)
    d_sums = hip.malloc(8 * n_sums)
    try:
        rc = L.nt_exec_replay_noalloc(x._h, d_in, paths, offset & 0xFFFFFFFFFFFFFFFF, seed, d_sums, n_sums, stream)
        if rc != 0:
            raise rocm.NtError(rc, L.nt_last_error().decode())
        if stream is None:
            hip.ok(hip.L.hipDeviceSynchronize())
        else:
            hip.ok(hip.L.hipStreamSynchronize(stream))
        return hip.to_host(d_sums, n_sums)
    finally:
        hip.L.hipFree(d_in)
        hip.L.hipFree(d_sums)


# (workload, precision, derivative mode, loop rolling, path counts of three consecutive
# calls). The reverse sweep (mode 1) keeps its tape per lane in device memory (288 bytes
# rolled, 272 bytes as a checkpointed straight line with roll -1), so its dispatches stay
# within the lanes whose tape fits the static array. 2,000,000 and 1,000,000 paths launch
# more blocks than the device holds (16 and 8 per CU).
CASES = [("C2", "fp64", 0, 1, (200_001, 4_097, 65_536)), ("C3", "fp32", 0, 1, (200_001, 4_097, 65_536)),
         ("C2", "fp64", 0, 1, (2_000_000, 4_097, 1_000_000)),
         ("C2", "fp64", 1, 1, (20_001, 4_097, 16_384)), ("C2", "fp64", 1, -1, (20_001, 4_097, 16_384))]


@pytest.mark.parametrize("name,prec,mode,roll,counts", CASES)
def test_noalloc_matches_replay(rocm, hip, tapes, name, prec, mode, roll, counts):
    t = tapes[name]
    recorded = np.asarray(t["recorded_inputs"], dtype=np.float64)
    moved = recorded.copy()
    moved[0] *= 1.05
    print(f"case noalloc {name} {prec} mode={mode} roll={roll}", flush=True)
    with rocm.Executable(t, rocm.options(prec, mode=mode, roll=roll)) as x:
        assert roll == 1 or x.info()["n_segments"] > 1
        # two calls in a row, the second smaller; then other inputs on a caller stream
        for paths, inputs, own_stream in zip(counts, (recorded, recorded, moved), (False, False, True)):
            x.set_inputs(inputs)
            want, _ = x.replay(paths, OFFSET, 42)
            x.set_inputs(recorded)
            stream = None
            if own_stream:
                s = C.c_void_p()
                hip.ok(hip.L.hipStreamCreate(C.byref(s)))
                stream = s
            try:
                got = noalloc(rocm, hip, x, inputs, paths, OFFSET, 42, stream)
            finally:
                if stream is not None:
                    hip.L.hipStreamDestroy(stream)
            print(f"  paths={paths} sum={got[0]!r}", flush=True)
            assert np.array_equal(got, want), (paths, got - want)


MERTON = dict(spot=100.0, strike=100.0, vol=0.18, rate=0.03, maturity=1.0, jumpIntensity=0.75, jumpMean=-0.05,
              jumpVol=0.15)


@pytest.mark.parametrize("mode,counts", [(2, (50_001, 4_097)), (1, (20_001, 4_097))])
def test_noalloc_with_exception_lanes(rocm, hip, nt, tapes, mode, counts):
    """The Merton jump tape (32 steps): its smoothed indicator overflows exp on
    most steps, so most lanes leave their paths to the exception kernel. Two
    calls in a row (the second smaller) are each bit-equal to nt_exec_replay's
    (which runs the exception kernel after a look at the count); then an
    executable whose lanes flag nothing (C2), on the same static array, is
    bit-equal too: the count and the lane bitmap were left at zero."""
    from conftest import merton_call_tape
    flat = merton_call_tape(nt, MERTON, steps=32).flat()
    print(f"case noalloc merton32 fp64 mode={mode}", flush=True)
    with rocm.Executable(flat, rocm.options("fp64", mode=mode)) as x:
        assert "nt_replay_slow" in x.source()
        for paths in counts:
            want, _ = x.replay(paths, OFFSET, 42)
            got = noalloc(rocm, hip, x, flat["recorded_inputs"], paths, OFFSET, 42)
            print(f"  paths={paths} sum={got[0]!r}", flush=True)
            assert np.all(np.isfinite(got))
            assert np.array_equal(got, want), (paths, got - want)
    t = tapes["C2"]
    with rocm.Executable(t, rocm.options("fp64")) as x:
        want, _ = x.replay(65_536, OFFSET, 42)
        got = noalloc(rocm, hip, x, t["recorded_inputs"], 65_536, OFFSET, 42)
    assert np.array_equal(got, want), got - want


@pytest.mark.parametrize("name,mode,paths", [("C2", 2, 200_001), ("C2", 2, 2_000_000), ("C3", 2, 100_000),
                                             ("C2", 1, 20_001), ("merton32", 2, 50_001)])
def test_noalloc_replays_from_a_captured_graph(rocm, hip, nt, tapes, name, mode, paths):
    """The entry point enqueues its kernels and nothing else (no allocation,
    copy, memset or wait), so a caller can capture it into a HIP graph: four
    launches of the instantiated graph, with eager replays and
    synchronisations between them, each give nt_exec_replay's sums for the
    same paths, offset and seed, bit for bit; also with a reverse sweep's
    device-memory tape and with lanes left to the exception kernel (the Merton
    tape), whose count and bitmap each launch leaves at zero."""
    L = hip.L
    if name == "merton32":
        from conftest import merton_call_tape
        t = merton_call_tape(nt, MERTON, steps=32).flat()
    else:
        t = tapes[name]
    print(f"case {name} mode={mode} paths={paths} noalloc captured into a graph", flush=True)
    with rocm.Executable(t, rocm.options("fp64", mode=mode)) as x:
        want, _ = x.replay(paths, OFFSET, 42)
        n_sums = x.n_outputs * (2 + x.n_inputs)
        d_in = hip.to_device(t["recorded_inputs"])
        d_sums = hip.malloc(8 * n_sums)
        stream, graph, gexec = C.c_void_p(), C.c_void_p(), C.c_void_p()
        hip.ok(L.hipStreamCreate(C.byref(stream)))
        try:
            hip.ok(L.hipStreamBeginCapture(stream, 2))  # hipStreamCaptureModeRelaxed
            rc = rocm.lib().nt_exec_replay_noalloc(x._h, d_in, paths, OFFSET, 42, d_sums, n_sums, stream)
            end = L.hipStreamEndCapture(stream, C.byref(graph))
            assert rc == 0, rocm.lib().nt_last_error().decode()
            assert end == 0, f"hipStreamEndCapture returned {end}"
            hip.ok(L.hipGraphInstantiate(C.byref(gexec), graph, None, None, 0))
            for i in range(4):
                hip.ok(L.hipMemset(d_sums, 0, 8 * n_sums))  # eager, outside the graph
                hip.ok(L.hipGraphLaunch(gexec, stream))
                hip.ok(L.hipStreamSynchronize(stream))
                got = hip.to_host(d_sums, n_sums)
                print(f"  launch {i}: sum={got[0]!r}", flush=True)
                assert np.array_equal(got, want), (i, got - want)
                x.replay(4_097, 0, 7)  # eager work on the executable's own stream
        finally:
            if gexec:
                L.hipGraphExecDestroy(gexec)
            if graph:
                L.hipGraphDestroy(graph)
            L.hipStreamDestroy(stream)
            L.hipFree(d_in)
            L.hipFree(d_sums)


def test_noalloc_refuses_oversized_scratch(rocm, hip, tapes):
    """A reverse-sweep executable that keeps its tape in device memory needs
    tape_slots x lanes of scratch; at the full grid that exceeds the static
    array, and the call is refused before anything is launched."""
    t = tapes["C2"]
    with rocm.Executable(t, rocm.options("fp64", mode=1, checkpoint=2)) as x:
        info = x.info()
        assert info["tape_slots"] > 0
        lanes = info["grid_cap"] * info["block"]
        assert info["tape_slots"] * 8 * lanes > (8 << 20)
        with pytest.raises(rocm.NtError) as e:
            noalloc(rocm, hip, x, t["recorded_inputs"], 2_000_000, 0, 42)
        assert e.value.status == rocm.NT_E_INVALID
        assert "scratch" in str(e.value)
