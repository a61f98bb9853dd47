"""Compile a generated replay kernel for the host (tests/host_emu) and run it.

Used only by the CPU tests of the lowering: the emitted source is built with
g++ -ffp-contract=off against glibc's libm, the same arithmetic as the oracle,
so fp64 per-path results can be compared to rounding level.
"""
from __future__ import annotations

import ctypes as C
import hashlib
import os
import subprocess
import tempfile
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parents[1]
EMU = Path(__file__).resolve().parent / "host_emu"
BUILD = Path(tempfile.gettempdir()) / "nt_host_emu"


class EmulatedKernel:
    def __init__(self, source: str, n_inputs: int, tape_slots: int, dump: bool = True):
        BUILD.mkdir(exist_ok=True)
        deps = "".join(p.read_text() for p in (EMU / "prelude.h", EMU / "emu_main.cpp",
                                                  ROOT / "nablatensor_amd" / "csrc" / "nt_skeleton.h",
                                                  ROOT / "nablatensor_amd" / "csrc" / "nt_math_tables.h"))
        key = hashlib.sha1((source + str(dump) + deps).encode()).hexdigest()[:16]
        src = BUILD / f"k_{key}.hip.h"
        so = BUILD / f"k_{key}.so"
        if not so.exists():
            src_tmp = Path(f"{src}.{os.getpid()}")
            src_tmp.write_text(source)
            os.replace(src_tmp, src)
            tmp = f"{so}.{os.getpid()}.tmp"  # test workers may build the same kernel at once
            cmd = ["g++", "-O1", "-std=c++17", "-shared", "-fPIC", "-ffp-contract=off", "-w",
                   f"-I{ROOT / 'nablatensor_amd' / 'csrc'}", f"-I{EMU}", f'-DNT_KERNEL_FILE="{src}"',
                   str(EMU / "emu_main.cpp"), "-o", tmp]
            if dump:
                cmd.insert(1, "-DNT_DUMP_PATHS=1")
            subprocess.run(cmd, check=True)
            os.replace(tmp, so)
        self.lib = C.CDLL(str(so))
        self.lib.emu_run.argtypes = [C.c_uint64, C.c_uint64, C.c_uint64, C.POINTER(C.c_double),
                                     C.POINTER(C.c_double), C.POINTER(C.c_double), C.POINTER(C.c_double),
                                     C.c_uint, C.c_uint, C.c_ulonglong]
        self.n_inputs = n_inputs
        self.slots = tape_slots

    def run(self, inputs, paths: int, offset: int = 0, seed: int = 42, grid: int = 4, block: int = 64,
            markets: int = 1, outputs: int = 1):
        """One emulated dispatch. With markets > 1, `inputs` holds one row per
        market and every result gains a leading market axis; with outputs > 1,
        per-path rows gain an output axis after the path and sums hold one
        row per output."""
        x = np.ascontiguousarray(inputs, dtype=np.float64).reshape(-1)
        ni = self.n_inputs
        sums = np.zeros(markets * outputs * (2 + ni))
        values = np.zeros(markets * paths * outputs)
        grads = np.zeros((markets * paths * outputs, max(1, ni)))
        p = lambda a: a.ctypes.data_as(C.POINTER(C.c_double))
        rc = self.lib.emu_run(paths, offset & (2**64 - 1), seed & (2**64 - 1), p(x), p(sums), p(values), p(grads),
                              grid, block, self.slots)
        if rc != 0:
            raise AssertionError("the exception kernel left lane flags set")
        grads = grads[:, :ni]
        if outputs > 1:
            sums = sums.reshape(markets, outputs, 2 + ni)
            values = values.reshape(markets, paths, outputs)
            grads = grads.reshape(markets, paths, outputs, ni)
            return (sums[0], values[0], grads[0]) if markets == 1 else (sums, values, grads)
        if markets == 1:
            return sums, values, grads
        return (sums.reshape(markets, 2 + ni), values.reshape(markets, paths),
                grads.reshape(markets, paths, ni))
