"""The lowering (tape validation, planning, source emission) and the CPU
oracle under AddressSanitizer and UndefinedBehaviorSanitizer, on the CPU.

tests/sanitize/Makefile builds lower.cpp and oracle/nt_oracle.c with
-fsanitize=address,undefined (host code only, no GPU code) into a driver
that reads tapes in the C ABI's wire form. It lowers every valid tape under
a spread of options (both precisions, both derivative modes, the three
checkpoint policies, rolled and straight-line, segment lengths, several
markets, both tangent bases, contraction and Box-Muller variants), replays
it in the oracle, and checks that build_ir refuses each malformed tape with
an error: unknown opcodes, operands that are not earlier nodes, bad draw
ordinals and streams, input lists that do not match the INPUT nodes,
outputs out of range, no streams, empty tapes, null arrays. Any sanitizer
report fails the run.
"""
from __future__ import annotations

import subprocess

import numpy as np
import pytest

from conftest import ROOT, asian_tape, branching_tape, merton_call_tape, random_tape, two_output_tape

SAN = ROOT / "tests" / "sanitize"


def wire(flat: dict) -> bytes:
    from nablatensor_amd import rocm
    return rocm.TapeArrays(flat).wire_bytes()


def malformed(flat: dict) -> list[dict]:
    """Copies of a valid tape, each broken in one way build_ir must refuse."""
    n = len(flat["op"])
    out = []

    def edit(**kw):
        f = {k: (list(v) if isinstance(v, (list, tuple, np.ndarray)) else v) for k, v in flat.items()}
        for k, fn in kw.items():
            fn(f)
        out.append(f)

    first_binary = next(i for i, op in enumerate(flat["op"]) if op in (4, 5, 6, 7, 12, 13))
    first_draw = next(i for i, op in enumerate(flat["op"]) if op in (2, 3))
    first_input = flat["input_node"][0]
    edit(op=lambda f: f["op"].__setitem__(first_binary, 15))
    edit(op=lambda f: f["op"].__setitem__(first_binary, -1))
    edit(a=lambda f: f["arg_a"].__setitem__(first_binary, first_binary))
    edit(a=lambda f: f["arg_a"].__setitem__(first_binary, -3))
    edit(b=lambda f: f["arg_b"].__setitem__(first_binary, n + 5))
    edit(d=lambda f: f["arg_a"].__setitem__(first_draw, -1))
    edit(d=lambda f: f["arg_b"].__setitem__(first_draw, 7))
    edit(s=lambda f: f.__setitem__("n_streams", 0))
    edit(i=lambda f: f["arg_a"].__setitem__(first_input, 99))
    edit(i=lambda f: f["input_node"].__setitem__(0, first_binary))
    edit(i=lambda f: f["input_node"].__setitem__(0, -1))
    edit(o=lambda f: f["output_node"].__setitem__(0, n))
    edit(o=lambda f: f["output_node"].__setitem__(0, -1))
    edit(o=lambda f: f.__setitem__("output_node", []))
    edit(e=lambda f: [f.__setitem__(k, []) for k in ("op", "arg_a", "arg_b", "constant")])
    return out


def test_lowering_and_oracle_under_sanitizers(nt, tapes, tmp_path):
    build = subprocess.run(["make", "-s", "-C", str(SAN)], capture_output=True, text=True)
    assert build.returncode == 0, build.stdout + build.stderr
    from nablatensor_amd import workloads
    valid = dict(tapes)
    valid["weekdays"] = workloads.schedule_tapes()["asian_weekdays"].flat()
    valid["asian96"] = asian_tape(nt, 96).flat()
    valid["branching"] = branching_tape(nt).flat()
    valid["merton"] = merton_call_tape(nt, dict(spot=100.0, strike=100.0, vol=0.18, rate=0.03, maturity=1.0,
                                                jumpIntensity=0.75, jumpMean=-0.05, jumpVol=0.15), steps=24).flat()
    valid["two_outputs"] = two_output_tape(nt).flat()
    for seed in range(6):
        valid[f"random{seed}"] = random_tape(nt, seed, 40 + 60 * seed).flat()
    lines = []
    for name, flat in valid.items():
        p = tmp_path / f"{name}.bin"
        p.write_bytes(wire(flat))
        lines.append(f"{p} ok")
    bad = malformed(tapes["C2"]) + malformed(valid["random1"])
    for k, flat in enumerate(bad):
        p = tmp_path / f"bad{k}.bin"
        p.write_bytes(wire(flat))
        lines.append(f"{p} invalid")
    manifest = tmp_path / "manifest.txt"
    manifest.write_text("\n".join(lines) + "\n")
    run = subprocess.run([str(SAN / "_build" / "nt_sanitize_driver"), str(manifest)], capture_output=True, text=True,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0:halt_on_error=1",
                              "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1", "PATH": "/usr/bin:/bin"},
                         timeout=900)
    print(run.stdout[-2000:])
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-8000:]
    assert f"tapes {len(lines)}, refused {len(bad)}, failures 0" in run.stdout
