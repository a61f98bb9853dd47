"""ctypes binding of the C ABI in include/nablatensor_rocm.h (libnt_rocm.so).

The same symbols a Java FFM adapter binds; tests and bench.py go through this
module so that what they exercise is the C ABI itself. The library must have
been built in-tree (nablatensor_amd/build.py); nothing falls back to a CPU
path when it is missing.
"""
from __future__ import annotations

import ctypes as C
from pathlib import Path

import numpy as np

LIB_PATH = Path(__file__).resolve().parent / "libnt_rocm.so"

NT_OK = 0
NT_E_INVALID, NT_E_UNSUPPORTED, NT_E_NO_DEVICE, NT_E_COMPILE, NT_E_CLOSED, NT_E_INTERNAL = -1, -2, -3, -4, -5, -6
NT_FP64, NT_FP32 = 0, 1
NT_CKPT_AUTO, NT_CKPT_RECOMPUTE, NT_CKPT_STORE_DRAWS, NT_CKPT_STORE_ALL = 0, 1, 2, 3
NT_MODE_AUTO, NT_MODE_REVERSE, NT_MODE_TANGENT = 0, 1, 2
ABI_VERSION = 3

EXPORTS = ("nt_probe", "nt_device_name", "nt_lower", "nt_compile_check", "nt_exec_create", "nt_exec_set_inputs",
           "nt_exec_replay", "nt_exec_replay_many", "nt_exec_replay_paths", "nt_exec_replay_noalloc",
           "nt_exec_info_get", "nt_exec_grid", "nt_exec_source",
           "nt_exec_destroy", "nt_last_error", "nt_abi_version")


class NtTape(C.Structure):
    _fields_ = [("n_nodes", C.c_int32), ("op", C.POINTER(C.c_int32)), ("arg_a", C.POINTER(C.c_int32)),
                ("arg_b", C.POINTER(C.c_int32)), ("constant", C.POINTER(C.c_double)), ("n_inputs", C.c_int32),
                ("input_node", C.POINTER(C.c_int32)), ("n_outputs", C.c_int32),
                ("output_node", C.POINTER(C.c_int32)), ("n_streams", C.c_int32), ("n_uniforms", C.c_int32)]


class NtOptions(C.Structure):
    _fields_ = [("precision", C.c_int32), ("adjoints", C.c_int32), ("block", C.c_int32),
                ("max_blocks", C.c_int32), ("checkpoint", C.c_int32), ("seg_len", C.c_int32),
                ("roll", C.c_int32), ("contract", C.c_int32), ("libm", C.c_int32), ("mode", C.c_int32),
                ("markets", C.c_int32), ("waves", C.c_int32), ("basis", C.c_int32),
                ("allow_spill", C.c_int32), ("reserved", C.c_int32 * 2)]


class NtExecInfo(C.Structure):
    _fields_ = [(name, C.c_int32) for name in (
        "n_nodes", "n_active", "n_inputs", "n_channels", "loop_start", "loop_period", "loop_iters",
        "loop_carries", "seg_len", "n_segments", "checkpoint", "tape_slots", "vgprs", "sgprs", "agprs",
        "scratch_bytes", "lds_bytes", "block", "grid_cap", "mode")] + [("compile_seconds", C.c_double)]

    def as_dict(self) -> dict:
        return {name: getattr(self, name) for name, _ in self._fields_}


class NtError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"[{status}] {message}")
        self.status = status


_lib = None


def lib() -> C.CDLL:
    """Load libnt_rocm.so; raises if it has not been built."""
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise ImportError(f"{LIB_PATH} is missing: run `python -c 'import __graft_entry__ as g; g.build()'` "
                              "or `python nablatensor_amd/build.py` first")
        L = C.CDLL(str(LIB_PATH))
        L.nt_last_error.restype = C.c_char_p
        L.nt_probe.argtypes = [C.POINTER(C.c_int32)]
        L.nt_device_name.argtypes = [C.c_char_p, C.c_int32, C.c_char_p, C.c_int32]
        L.nt_lower.argtypes = [C.POINTER(NtTape), C.POINTER(NtOptions), C.c_char_p, C.POINTER(C.c_int64)]
        L.nt_compile_check.argtypes = [C.POINTER(NtTape), C.POINTER(NtOptions), C.POINTER(NtExecInfo)]
        L.nt_exec_create.argtypes = [C.POINTER(NtTape), C.POINTER(NtOptions), C.POINTER(C.c_void_p)]
        L.nt_exec_set_inputs.argtypes = [C.c_void_p, C.POINTER(C.c_double), C.c_int32]
        L.nt_exec_replay.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(C.c_double),
                                     C.c_int32, C.POINTER(C.c_double)]
        L.nt_exec_replay_many.argtypes = [C.c_void_p, C.POINTER(C.c_double), C.c_int32, C.c_uint64, C.c_uint64,
                                          C.c_uint64, C.POINTER(C.c_double), C.c_int32, C.POINTER(C.c_double)]
        L.nt_exec_replay_paths.argtypes = [C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64,
                                           C.POINTER(C.c_double), C.POINTER(C.c_double)]
        L.nt_exec_replay_noalloc.argtypes = [C.c_void_p, C.c_void_p, C.c_uint64, C.c_uint64, C.c_uint64,
                                             C.c_void_p, C.c_int32, C.c_void_p]
        L.nt_exec_info_get.argtypes = [C.c_void_p, C.POINTER(NtExecInfo)]
        L.nt_exec_grid.argtypes = [C.c_void_p, C.c_uint64, C.POINTER(C.c_int32), C.POINTER(C.c_int32)]
        L.nt_exec_source.argtypes = [C.c_void_p, C.c_char_p, C.POINTER(C.c_int64)]
        L.nt_exec_destroy.argtypes = [C.c_void_p]
        if L.nt_abi_version() != ABI_VERSION:
            raise ImportError(f"{LIB_PATH} has ABI version {L.nt_abi_version()}, this binding expects {ABI_VERSION}: "
                              "rebuild it")
        _lib = L
    return _lib


def _check(status: int) -> None:
    if status != NT_OK:
        raise NtError(status, lib().nt_last_error().decode(errors="replace"))


class TapeArrays:
    """Keeps the numpy arrays of a flat tape alive while an NtTape points at them."""

    def __init__(self, flat: dict):
        self.op = np.ascontiguousarray(flat["op"], dtype=np.int32)
        self.arg_a = np.ascontiguousarray(flat["arg_a"], dtype=np.int32)
        self.arg_b = np.ascontiguousarray(flat["arg_b"], dtype=np.int32)
        self.constant = np.ascontiguousarray(flat["constant"], dtype=np.float64)
        self.input_node = np.ascontiguousarray(flat["input_node"], dtype=np.int32)
        self.output_node = np.ascontiguousarray(flat["output_node"], dtype=np.int32)
        self.n_streams = int(flat.get("n_streams", 1))
        self.n_uniforms = int(flat.get("n_uniforms", 0))

    def wire_bytes(self) -> bytes:
        """The tape's canonical byte form: the nt_tape fields in struct order,
        little-endian (int32 counts and indices, IEEE-754 binary64 constants):
        n_nodes, op, arg_a, arg_b, constant, n_inputs, input_node, n_outputs,
        output_node, n_streams, n_uniforms. These are FlatTape's arrays
        (FlatTape.java:37-79) minus `active`, which the engine derives itself;
        a foreign-function adapter hashes the same bytes of what it marshals."""
        i32 = lambda v: np.asarray(v, dtype="<i4").tobytes()
        n = len(self.op)
        return b"".join([i32([n]), i32(self.op), i32(self.arg_a), i32(self.arg_b),
                         np.asarray(self.constant, dtype="<f8").tobytes(), i32([len(self.input_node)]),
                         i32(self.input_node), i32([len(self.output_node)]), i32(self.output_node),
                         i32([self.n_streams, self.n_uniforms])])

    def struct(self) -> NtTape:
        p32 = lambda a: a.ctypes.data_as(C.POINTER(C.c_int32))
        return NtTape(len(self.op), p32(self.op), p32(self.arg_a), p32(self.arg_b),
                      self.constant.ctypes.data_as(C.POINTER(C.c_double)), len(self.input_node),
                      p32(self.input_node), len(self.output_node), p32(self.output_node),
                      self.n_streams, self.n_uniforms)


def wire_digest(flat: dict) -> str:
    """SHA-256 (hex) of TapeArrays.wire_bytes: the identity of a tape as it
    crosses the C ABI."""
    import hashlib

    return hashlib.sha256(TapeArrays(flat).wire_bytes()).hexdigest()


def options(precision: str = "fp64", adjoints: bool = True, block: int = 0, max_blocks: int = 0,
            checkpoint: int = NT_CKPT_AUTO, seg_len: int = 0, roll: int = 1, contract: int = 0,
            libm: int = 0, mode: int = 0, markets: int = 0, waves: int = 0, basis: int = 0,
            allow_spill: bool = False) -> NtOptions:
    return NtOptions(NT_FP32 if precision == "fp32" else NT_FP64, 1 if adjoints else 0, block, max_blocks,
                     checkpoint, seg_len, roll, contract, libm, mode, markets, waves, basis, int(allow_spill))


def probe() -> int:
    n = C.c_int32(0)
    _check(lib().nt_probe(C.byref(n)))
    return n.value


def device_name() -> tuple[str, str]:
    name = C.create_string_buffer(256)
    arch = C.create_string_buffer(64)
    _check(lib().nt_device_name(name, 256, arch, 64))
    return name.value.decode(), arch.value.decode()


def lower(flat: dict, opts: NtOptions | None = None) -> str:
    arrays = TapeArrays(flat)
    t = arrays.struct()
    o = opts or options()
    n = C.c_int64(0)
    _check(lib().nt_lower(C.byref(t), C.byref(o), None, C.byref(n)))
    buf = C.create_string_buffer(n.value)
    _check(lib().nt_lower(C.byref(t), C.byref(o), buf, C.byref(n)))
    return buf.value.decode()


def compile_check(flat: dict, opts: NtOptions | None = None) -> dict:
    arrays = TapeArrays(flat)
    t = arrays.struct()
    o = opts or options()
    info = NtExecInfo()
    _check(lib().nt_compile_check(C.byref(t), C.byref(o), C.byref(info)))
    return info.as_dict()


class Executable:
    """One nt_exec: a lowered, compiled and loaded tape."""

    def __init__(self, flat: dict, opts: NtOptions | None = None):
        arrays = TapeArrays(flat)
        t = arrays.struct()
        self.options = opts or options()
        self.n_inputs = len(arrays.input_node)
        self.n_outputs = len(arrays.output_node)
        h = C.c_void_p()
        _check(lib().nt_exec_create(C.byref(t), C.byref(self.options), C.byref(h)))
        self._h = h

    def set_inputs(self, values) -> None:
        v = np.ascontiguousarray(values, dtype=np.float64)
        _check(lib().nt_exec_set_inputs(self._h, v.ctypes.data_as(C.POINTER(C.c_double)), len(v)))

    def replay(self, paths: int, offset: int = 0, seed: int = 42):
        """Raw sums [sum y, sum y^2, sum adjoints...] (one such row per output,
        concatenated) and timing {kernel_ms, wall_ms, replay_ms}."""
        sums = np.zeros(self.n_outputs * (2 + self.n_inputs), dtype=np.float64)
        timing = np.zeros(3, dtype=np.float64)
        _check(lib().nt_exec_replay(self._h, paths, offset & 0xFFFFFFFFFFFFFFFF, seed & 0xFFFFFFFFFFFFFFFF,
                                    sums.ctypes.data_as(C.POINTER(C.c_double)), len(sums),
                                    timing.ctypes.data_as(C.POINTER(C.c_double))))
        return sums, {"kernel_ms": timing[0], "wall_ms": timing[1], "replay_ms": timing[2]}

    def replay_many(self, input_sets, paths: int, offset: int = 0, seed: int = 42):
        """Raw sums per input set, shape (markets, 2 + n_inputs), from one dispatch
        that shares each path's draws across the sets; and timing as replay()."""
        x = np.ascontiguousarray(input_sets, dtype=np.float64)
        markets = x.shape[0] if x.ndim == 2 else 1
        if x.size != markets * self.n_inputs:
            raise ValueError(f"expected {markets} x {self.n_inputs} input values, got shape {x.shape}")
        sums = np.zeros((markets, self.n_outputs * (2 + self.n_inputs)), dtype=np.float64)
        timing = np.zeros(3, dtype=np.float64)
        _check(lib().nt_exec_replay_many(self._h, x.ctypes.data_as(C.POINTER(C.c_double)), markets, paths,
                                         offset & 0xFFFFFFFFFFFFFFFF, seed & 0xFFFFFFFFFFFFFFFF,
                                         sums.ctypes.data_as(C.POINTER(C.c_double)), sums.size,
                                         timing.ctypes.data_as(C.POINTER(C.c_double))))
        return sums, {"kernel_ms": timing[0], "wall_ms": timing[1], "replay_ms": timing[2]}

    def replay_paths(self, paths: int, offset: int = 0, seed: int = 42):
        """Per-path values (paths,) and derivatives (paths, inputs); with
        several outputs (paths, outputs) and (paths, outputs, inputs)."""
        no = self.n_outputs
        values = np.zeros(paths * no, dtype=np.float64)
        grads = np.zeros((paths * no, max(1, self.n_inputs)), dtype=np.float64)
        _check(lib().nt_exec_replay_paths(self._h, paths, offset & 0xFFFFFFFFFFFFFFFF, seed & 0xFFFFFFFFFFFFFFFF,
                                          values.ctypes.data_as(C.POINTER(C.c_double)),
                                          grads.ctypes.data_as(C.POINTER(C.c_double))))
        grads = grads[:, :self.n_inputs]
        if no == 1:
            return values, grads
        return values.reshape(paths, no), grads.reshape(paths, no, self.n_inputs)

    def info(self) -> dict:
        i = NtExecInfo()
        _check(lib().nt_exec_info_get(self._h, C.byref(i)))
        return i.as_dict()

    def grid(self, paths: int) -> tuple[int, int]:
        """(blocks, threads per block) of a single-set dispatch of `paths`."""
        g, b = C.c_int32(0), C.c_int32(0)
        _check(lib().nt_exec_grid(self._h, paths, C.byref(g), C.byref(b)))
        return g.value, b.value

    def source(self) -> str:
        n = C.c_int64(0)
        _check(lib().nt_exec_source(self._h, None, C.byref(n)))
        buf = C.create_string_buffer(n.value)
        _check(lib().nt_exec_source(self._h, buf, C.byref(n)))
        return buf.value.decode()

    def close(self) -> None:
        if self._h:
            lib().nt_exec_destroy(self._h)
            self._h = C.c_void_p()

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
