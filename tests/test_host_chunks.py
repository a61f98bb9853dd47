"""The host layer's chunked replay on the CPU (a failure-path check with a
tiny chunk budget), under AddressSanitizer and UndefinedBehaviorSanitizer.

tests/host_chunks/driver.cpp drives AadExecutable::calibrate / replaySafe
(nablatensor_amd/host/engine.cpp) with a stand-in executable that sums a
fixed function of the path index and reports a chosen rate of 10^8 paths/s:

* calibration probes 65,536 paths (AbstractAadExecutable.java:124-139), then
  chunks of rate x budget paths, at least 4,096;
* chunks that carry raw sums combine exactly into one replay's result;
  chunks that carry means only combine by the reference's mean x n
  reconstruction (AadResultAccumulator.java:52-96);
* a non-positive budget or path count is an IllegalArgumentException
  (std::invalid_argument) and a closed executable an IllegalStateException
  (std::logic_error), as AbstractAadExecutable.java:87-98 and
  DeviceAadExecutable.java:142-144 have them.
"""
from __future__ import annotations

import json
import subprocess

import pytest

from conftest import ROOT

DIR = ROOT / "tests" / "host_chunks"


def test_chunked_replay_under_sanitizers():
    build = subprocess.run(["make", "-s", "-C", str(DIR)], capture_output=True, text=True)
    assert build.returncode == 0, build.stdout + build.stderr
    run = subprocess.run([str(DIR / "_build" / "nt_chunk_driver")], capture_output=True, text=True, timeout=300,
                         env={"ASAN_OPTIONS": "detect_leaks=1:abort_on_error=0:halt_on_error=1",
                              "UBSAN_OPTIONS": "print_stacktrace=1:halt_on_error=1", "PATH": "/usr/bin:/bin"})
    assert run.returncode == 0, run.stdout[-4000:] + run.stderr[-8000:]
    cases = {c["case"]: c for c in (json.loads(line) for line in run.stdout.splitlines())}

    # chunks that carry raw sums combine exactly into one replay's result
    c = cases["raw"]
    assert c["chunks"] == 1 + 30 and c["first_chunks"] == [65536] + [100000] * 5
    assert c["rate"] == 1e8 and c["paths"] == 3_000_000
    assert c["value"][0] == pytest.approx(c["value"][1], rel=1e-15)
    assert c["grad0"][0] == pytest.approx(c["grad0"][1], rel=1e-15)
    assert c["stderr"][0] == pytest.approx(c["stderr"][1], rel=1e-12)
    assert c["seconds"] == pytest.approx(0.03, rel=1e-12)  # the chunks' time, the probe excluded

    # chunks with means only: the reference's mean x n reconstruction
    c = cases["means"]
    assert c["chunks"] == 31
    assert c["value"][0] == pytest.approx(c["value"][1], rel=1e-14)
    assert c["grad0"][0] == pytest.approx(c["grad0"][1], rel=1e-14)
    assert c["stderr"][0] == pytest.approx(c["stderr"][1], rel=1e-10)

    # a budget below the minimum chunk: chunks of 4,096 paths
    c = cases["min_chunk"]
    assert c["first_chunks"] == [65536] + [4096] * 5
    assert c["chunks"] == 1 + 25  # 24 x 4,096 + 1,696
    assert c["value"][0] == pytest.approx(c["value"][1], rel=1e-14)

    # a non-positive budget or path count, and a closed executable, are refused
    assert cases["refusals"]["refused"] == 3
