"""ctypes wrapper of the CPU oracle (libnt_oracle.so) — TEST INFRASTRUCTURE ONLY.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import
this module. It restates the reference's scalar `cpu` engine (see nt_oracle.h
for the file:line each function follows); the tests hold the HIP engine to it,
and it is never a fallback for it.
"""
from __future__ import annotations

import contextlib
import ctypes as C
import subprocess
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libnt_oracle.so"


class _Tape(C.Structure):
    _fields_ = [("n", C.c_int32), ("op", C.POINTER(C.c_int32)), ("arg_a", C.POINTER(C.c_int32)),
                ("arg_b", C.POINTER(C.c_int32)), ("constant", C.POINTER(C.c_double)), ("n_inputs", C.c_int32),
                ("input_node", C.POINTER(C.c_int32)), ("n_outputs", C.c_int32),
                ("output_node", C.POINTER(C.c_int32)), ("n_streams", C.c_int32)]


class _Totals(C.Structure):
    _fields_ = [("value", C.POINTER(C.c_double)), ("sumsq", C.POINTER(C.c_double)),
                ("gradient", C.POINTER(C.c_double))]


_lib = None


def lib() -> C.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
        _lib = _bind(C.CDLL(str(LIB_PATH)))
    return _lib


def build_planted(plant: int, out: Path) -> Path:
    """Builds the oracle with planted mistake `plant` (NTO_PLANT in
    nt_oracle.c: reverse rule `plant` made wrong) into `out`."""
    subprocess.run(["make", "-s", "-C", str(HERE), "planted", f"PLANT={int(plant)}", f"OUT={out}"], check=True)
    return Path(out)


@contextlib.contextmanager
def library(path):
    """Every call inside the block goes to the oracle build at `path` (a
    planted-mistake build from build_planted); the default build after it."""
    global _lib
    saved = _lib
    _lib = _bind(C.CDLL(str(path)))
    try:
        yield
    finally:
        _lib = saved


def _bind(L: C.CDLL) -> C.CDLL:
    L.nto_philox2x32_10.argtypes = [C.c_uint32, C.c_uint32, C.c_uint32, C.POINTER(C.c_uint32)]
    L.nto_normal.argtypes = [C.c_uint64, C.c_uint64, C.c_int32, C.c_int32]
    L.nto_normal.restype = C.c_double
    L.nto_uniform.argtypes = [C.c_uint64, C.c_uint64, C.c_int32, C.c_int32]
    L.nto_uniform.restype = C.c_double
    L.nto_mark_active.argtypes = [C.POINTER(_Tape), C.POINTER(C.c_uint8)]
    L.nto_replay.argtypes = [C.POINTER(_Tape), C.POINTER(C.c_double), C.c_uint64, C.c_uint64, C.c_uint64,
                             C.c_int, C.c_int, C.c_int, C.POINTER(_Totals)]
    L.nto_replay_paths.argtypes = [C.POINTER(_Tape), C.POINTER(C.c_double), C.c_uint64, C.c_uint64,
                                   C.c_uint64, C.c_int, C.c_int, C.POINTER(C.c_double),
                                   C.POINTER(C.c_double)]
    L.nto_replay_paths_perturbed.argtypes = [C.POINTER(_Tape), C.POINTER(C.c_double), C.c_uint64, C.c_uint64,
                                             C.c_uint64, C.c_int, C.c_uint64, C.POINTER(C.c_double),
                                             C.POINTER(C.c_double)]
    return L


class Tape:
    """A flat tape (the dict of AadTape.flat() or the same keys) pinned for C."""

    def __init__(self, flat: dict):
        self.op = np.ascontiguousarray(flat["op"], dtype=np.int32)
        self.arg_a = np.ascontiguousarray(flat["arg_a"], dtype=np.int32)
        self.arg_b = np.ascontiguousarray(flat["arg_b"], dtype=np.int32)
        self.constant = np.ascontiguousarray(flat["constant"], dtype=np.float64)
        self.input_node = np.ascontiguousarray(flat["input_node"], dtype=np.int32)
        self.output_node = np.ascontiguousarray(flat["output_node"], dtype=np.int32)
        self.n_streams = int(flat.get("n_streams", 1))
        self.recorded = np.ascontiguousarray(flat.get("recorded_inputs", self.constant[self.input_node]),
                                             dtype=np.float64)
        p = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))
        self.s = _Tape(len(self.op), p(self.op), p(self.arg_a), p(self.arg_b),
                       self.constant.ctypes.data_as(C.POINTER(C.c_double)), len(self.input_node),
                       p(self.input_node), len(self.output_node), p(self.output_node), self.n_streams)

    @property
    def n_inputs(self) -> int:
        return len(self.input_node)


def philox(c0: int, c1: int, key: int) -> tuple[int, int]:
    out = (C.c_uint32 * 2)()
    lib().nto_philox2x32_10(c0, c1, key, out)
    return out[0], out[1]


def normal(path: int, seed: int, k: int, stream: int = 0) -> float:
    return lib().nto_normal(path & (2**64 - 1), seed & (2**64 - 1), stream, k)


def uniform(path: int, seed: int, k: int, stream: int = 0) -> float:
    return lib().nto_uniform(path & (2**64 - 1), seed & (2**64 - 1), stream, k)


def active(flat: dict) -> np.ndarray:
    t = Tape(flat)
    out = np.zeros(len(t.op), dtype=np.uint8)
    lib().nto_mark_active(C.byref(t.s), out.ctypes.data_as(C.POINTER(C.c_uint8)))
    return out


def replay_sums(flat: dict, paths: int, offset: int = 0, seed: int = 42, inputs=None, f32: bool = False,
                adjoints: bool = True, threads: int = 0, all_outputs: bool = False) -> np.ndarray:
    """Raw sums [sum y, sum y^2, sum adjoint_j...] for output 0 (AadTotals
    fields); with all_outputs, one such row per output, concatenated."""
    t = Tape(flat)
    x = np.ascontiguousarray(t.recorded if inputs is None else inputs, dtype=np.float64)
    no = len(t.output_node)
    val = np.zeros(no)
    sq = np.zeros(no)
    gr = np.zeros(no * max(1, t.n_inputs))
    tot = _Totals(val.ctypes.data_as(C.POINTER(C.c_double)), sq.ctypes.data_as(C.POINTER(C.c_double)),
                  gr.ctypes.data_as(C.POINTER(C.c_double)))
    rc = lib().nto_replay(C.byref(t.s), x.ctypes.data_as(C.POINTER(C.c_double)), paths,
                          offset & (2**64 - 1), seed & (2**64 - 1), int(f32), int(adjoints), threads, C.byref(tot))
    if rc != 0:
        raise ValueError(f"oracle rejected the tape ({rc})")
    ni = t.n_inputs
    rows = [np.concatenate([[val[o], sq[o]], gr[o * ni:(o + 1) * ni]]) for o in range(no if all_outputs else 1)]
    return np.concatenate(rows)


def replay_paths(flat: dict, paths: int, offset: int = 0, seed: int = 42, inputs=None, f32: bool = False,
                 threads: int = 0, output=0, perturb: int = 0) -> tuple[np.ndarray, np.ndarray]:
    """Per-path value and adjoints of output `output` (None: every output,
    shapes (paths, outputs) and (paths, outputs, inputs)). perturb != 0 (fp64
    only) moves every transcendental result by one unit in the fixed
    pseudo-random pattern `perturb` (nto_replay_paths_perturbed)."""
    t = Tape(flat)
    x = np.ascontiguousarray(t.recorded if inputs is None else inputs, dtype=np.float64)
    no = len(t.output_node)
    values = np.zeros((paths, no))
    grads = np.zeros((paths, no, max(1, t.n_inputs)))
    if perturb:
        if f32:
            raise ValueError("perturbed replays are fp64")
        rc = lib().nto_replay_paths_perturbed(C.byref(t.s), x.ctypes.data_as(C.POINTER(C.c_double)), paths,
                                              offset & (2**64 - 1), seed & (2**64 - 1), threads, perturb,
                                              values.ctypes.data_as(C.POINTER(C.c_double)),
                                              grads.ctypes.data_as(C.POINTER(C.c_double)))
    else:
        rc = lib().nto_replay_paths(C.byref(t.s), x.ctypes.data_as(C.POINTER(C.c_double)), paths,
                                    offset & (2**64 - 1), seed & (2**64 - 1), int(f32), threads,
                                    values.ctypes.data_as(C.POINTER(C.c_double)),
                                    grads.ctypes.data_as(C.POINTER(C.c_double)))
    if rc != 0:
        raise ValueError(f"oracle rejected the tape ({rc})")
    grads = grads[:, :, :t.n_inputs]
    if output is None:
        return values, grads
    return values[:, output].copy(), grads[:, output, :].copy()


def to_result_c(sums: np.ndarray, paths: int, n_inputs: int) -> dict:
    """nto_to_result (the C restatement of AadTotals.toResult) for one output."""
    L = lib()
    L.nto_to_result.argtypes = [C.POINTER(_Totals), C.c_int32, C.c_int32, C.c_uint64, C.POINTER(C.c_double),
                                C.POINTER(C.c_double), C.POINTER(C.c_double)]
    val = np.array([sums[0]], dtype=np.float64)
    sq = np.array([sums[1]], dtype=np.float64)
    gr = np.ascontiguousarray(sums[2:2 + n_inputs], dtype=np.float64)
    tot = _Totals(val.ctypes.data_as(C.POINTER(C.c_double)), sq.ctypes.data_as(C.POINTER(C.c_double)),
                  gr.ctypes.data_as(C.POINTER(C.c_double)))
    mean, se, mg = np.zeros(1), np.zeros(1), np.zeros(max(1, n_inputs))
    L.nto_to_result(C.byref(tot), 1, n_inputs, paths, mean.ctypes.data_as(C.POINTER(C.c_double)),
                    se.ctypes.data_as(C.POINTER(C.c_double)), mg.ctypes.data_as(C.POINTER(C.c_double)))
    return {"price": float(mean[0]), "stderr": float(se[0]), "gradient": mg[:n_inputs]}


def to_result(sums: np.ndarray, paths: int) -> dict:
    """AadTotals.toResult (AadTotals.java:68-89): mean, stderr, mean gradient."""
    n = float(paths)
    mean = sums[0] / n
    if paths > 1:
        var = (sums[1] - n * mean * mean) / (n - 1.0)
        se = float(np.sqrt(max(0.0, var) / n))
    else:
        se = float("nan")
    return {"price": mean, "stderr": se, "gradient": np.asarray(sums[2:]) / n}


def path_errors(values, grads, ref_values, ref_grads):
    """Per path: value error |dv| / max(1, |v|) and normwise gradient error
    max_j |dg_j| / max(1, max_j |g_j|)."""
    def absdiff(a, b):
        # equal values (also equal infinities) and NaN against NaN count as
        # agreement; any other non-finite difference is an infinite error
        a, b = np.asarray(a, dtype=np.float64), np.asarray(b, dtype=np.float64)
        with np.errstate(invalid="ignore"):
            d = np.abs(a - b)
            d = np.where((a == b) | (np.isnan(a) & np.isnan(b)), 0.0, d)
        return np.where(np.isnan(d), np.inf, d)

    with np.errstate(invalid="ignore"):
        ev = absdiff(values, ref_values) / np.maximum(1.0, np.nan_to_num(np.abs(ref_values), nan=1.0))
        if not ref_grads.size:
            return ev, np.zeros(len(values))
        scale = np.maximum(1.0, np.nan_to_num(np.max(np.abs(ref_grads), axis=1), nan=1.0))
        eg = np.max(absdiff(grads, ref_grads), axis=1) / scale
    return ev, eg
