"""Failure paths the reference surfaces, forced from the host on the CPU.

* A hipRTC compile failure comes back as NT_E_COMPILE with hipRTC's log in
  nt_last_error, as the reference raises "hiprtcCompileProgram failed" with
  the program log (HipRuntime.java:351-354). The failure is made with the
  library's test-only hook (nablatensor_amd/csrc/nt_testing.h), which appends
  source that cannot compile to a real lowering.
* An engine library that cannot be loaded leaves the rocm engine discovered
  but unavailable, without throwing: isAvailable() is false
  (RocmAadEngine.java:53-59), AadEngines.available() leaves it out and
  select() fails with the reference's message (AadEngines.java:43-52,77-90),
  describe() says "no device", and compile() names the library it could not
  load. The library path is read once per process, so each case runs in a
  child process with NABLATENSOR_ROCM_LIB set.
"""
from __future__ import annotations

import ctypes as C
import json
import os
import subprocess
import sys

import pytest

from conftest import ROOT


@pytest.fixture()
def hook():
    from nablatensor_amd import rocm
    L = rocm.lib()
    L.nt_testing_append_source.argtypes = [C.c_char_p]
    L.nt_testing_append_source.restype = None
    yield L.nt_testing_append_source
    L.nt_testing_append_source(None)


def test_compile_failure_returns_the_hiprtc_log(tapes, hook):
    from nablatensor_amd import rocm
    hook(b"\n#error planted by the failure test\n")
    with pytest.raises(rocm.NtError) as e:
        rocm.compile_check(tapes["C1"], rocm.options("fp64"))
    assert e.value.status == rocm.NT_E_COMPILE
    msg = str(e.value)
    assert "hipRTC compile failed" in msg
    assert "planted by the failure test" in msg  # hipRTC's own log line
    hook(None)
    info = rocm.compile_check(tapes["C1"], rocm.options("fp64"))  # the hook is off again
    assert info["scratch_bytes"] == 0


def test_compile_failure_leaves_other_threads_alone(tapes, hook):
    """The hook is per thread: a compile on another thread is unaffected."""
    import threading
    from nablatensor_amd import rocm
    hook(b"\n#error planted by the failure test\n")
    out = {}

    def other():
        try:
            out["info"] = rocm.compile_check(tapes["C1"], rocm.options("fp64"))
        except Exception as exc:  # noqa: BLE001 - reported below
            out["error"] = exc

    t = threading.Thread(target=other)
    t.start()
    t.join()
    assert "error" not in out, out.get("error")
    assert out["info"]["scratch_bytes"] == 0


PROBE = r"""
import json, sys
sys.path.insert(0, {root!r})
import nablatensor_amd as nt
opts = nt.AadOptions.defaults()
rocm = [e for e in nt.AadEngines.discovered() if e.name() == "rocm"]
out = {{"discovered": [e.name() for e in nt.AadEngines.discovered()],
        "priority": rocm[0].priority(),
        "available": rocm[0].isAvailable(),
        "listed": [e.name() for e in nt.AadEngines.available(opts)],
        "describe": rocm[0].describe()}}
try:
    nt.AadEngines.select(opts)
    out["select"] = "returned"
except Exception as exc:
    out["select"] = str(exc)
try:
    nt.AadEngines.require("rocm", opts)
    out["require"] = "returned"
except Exception as exc:
    out["require"] = str(exc)
tape = nt.record(nt.Products.europeanCall(), nt.EquityMarket.atmOneYear(), nt.TimeGrid.uniform(1))
try:
    rocm[0].compile(tape, opts)
    out["compile"] = "returned"
except Exception as exc:
    out["compile"] = str(exc)
print(json.dumps(out))
"""


def probe(lib_path: str | None) -> dict:
    env = dict(os.environ)
    if lib_path is None:
        env.pop("NABLATENSOR_ROCM_LIB", None)
    else:
        env["NABLATENSOR_ROCM_LIB"] = lib_path
    env.pop("NABLATENSOR_ENGINE", None)
    r = subprocess.run([sys.executable, "-c", PROBE.format(root=str(ROOT))], env=env, capture_output=True, text=True,
                       timeout=120, check=True)
    return json.loads(r.stdout.strip().splitlines()[-1])


def test_missing_engine_library_is_unavailable_without_throwing(tmp_path):
    missing = str(tmp_path / "no-such-dir" / "libnt_rocm.so")
    out = probe(missing)
    assert out["discovered"] == ["rocm"] and out["priority"] == 55
    assert out["available"] is False
    assert "rocm" not in out["listed"]
    assert out["describe"] == "ROCm/HIP · no device"
    assert out["select"].startswith("no usable AAD engine; discovered: rocm")
    assert out["require"].startswith("AAD engine 'rocm' is not usable here; available: (none)")
    assert "no ROCm/HIP device available for the AAD replay kernel" in out["compile"]
    assert "cannot load " + missing in out["compile"]


def test_a_library_that_is_not_the_engine_is_unavailable():
    """A shared object that loads but lacks the nt_* entry points (the C math
    library) is refused the same way."""
    out = probe("libm.so.6")
    assert out["available"] is False and "rocm" not in out["listed"]
    assert "lacks an nt_* entry point" in out["compile"]


@pytest.mark.gpu
def test_executable_creation_reports_the_hiprtc_log_on_device(nt, tapes, hook):
    """On MI355X: nt_exec_create returns NT_E_COMPILE with the log, and the
    host layer (MonteCarlo ... .on("rocm").build()) raises it as a runtime
    error carrying the same log, as the reference's RuntimeException does;
    with the hook off the same tape builds and runs."""
    from nablatensor_amd import rocm
    assert rocm.probe() > 0, "no gfx950 device visible to libnt_rocm.so"
    print("case exec_create with a planted compile error", flush=True)
    hook(b"\n#error planted by the failure test\n")
    with pytest.raises(rocm.NtError) as e:
        rocm.Executable(tapes["C1"], rocm.options("fp64"))
    assert e.value.status == rocm.NT_E_COMPILE and "planted by the failure test" in str(e.value)
    builder = (nt.MonteCarlo.of(nt.Products.europeanCall()).market(nt.EquityMarket.atmOneYear())
               .steps(1).greeks().fp64().on("rocm"))
    with pytest.raises(RuntimeError) as e:
        builder.build()
    assert "hipRTC compile failed" in str(e.value) and "planted by the failure test" in str(e.value)
    hook(None)
    mc = builder.build()
    v = mc.run(100_000, 42)
    assert v.price() > 0
    mc.close()
