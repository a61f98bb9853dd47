"""The C ABI (include/nablatensor_rocm.h) without a GPU: exports, error codes,
the lowering entry points and offline hipRTC compilation for gfx950."""
from __future__ import annotations

import ctypes as C
import re
from pathlib import Path

import numpy as np
import pytest

from conftest import ROOT, gpu_available


@pytest.fixture(scope="module")
def rocm():
    from nablatensor_amd import rocm as r
    return r


def header_functions() -> list[str]:
    text = (ROOT / "include" / "nablatensor_rocm.h").read_text()
    return sorted(set(re.findall(r"^\s*(?:int|const char \*)\s*(nt_\w+)\(", text, re.M)))


def test_library_exports_every_declared_function(rocm):
    names = header_functions()
    assert len(names) >= 12
    lib = C.CDLL(str(rocm.LIB_PATH))
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(rocm.EXPORTS)
    assert lib.nt_abi_version() == 3


@pytest.mark.skipif(gpu_available(), reason="checks the no-device path")
def test_no_device_paths(rocm, tapes):
    assert rocm.probe() == 0
    with pytest.raises(rocm.NtError) as e:
        rocm.Executable(tapes["C1"])
    assert e.value.status == rocm.NT_E_NO_DEVICE
    assert "no ROCm/HIP gfx950 device" in str(e.value)


def _mutated(flat, **kw):
    out = {k: (np.array(v, copy=True) if isinstance(v, np.ndarray) else v) for k, v in flat.items()}
    out.update(kw)
    return out


def test_extended_tapes_lower_and_bad_draws_are_rejected(rocm, tapes):
    """Multi-output tapes, uniforms and named streams lower (the reference's
    device engines decline them, AadEngine.java:56-86; this one takes them);
    a multi-output tape refuses a forced reverse sweep; draws naming a stream
    the tape does not have are malformed."""
    flat = tapes["C1"]
    two_outputs = _mutated(flat, output_node=np.array([25, 24], dtype=np.int32))
    assert "mode=tangent" in rocm.lower(two_outputs)
    with pytest.raises(rocm.NtError) as e:
        rocm.lower(two_outputs, rocm.options(mode=rocm.NT_MODE_REVERSE))
    assert e.value.status == rocm.NT_E_UNSUPPORTED and "one output" in str(e.value)
    uniform = _mutated(flat)
    uniform["op"][14] = 3  # RANDU
    assert "nt_uniform(" in rocm.lower(uniform)
    streams = _mutated(flat, n_streams=2)
    streams["arg_b"][14] = 1
    assert "rhi1 = rhi ^ 0x9E3779B1u" in rocm.lower(streams)
    bad = _mutated(flat)
    bad["arg_b"][14] = 1  # stream 1 of a one-stream tape
    with pytest.raises(rocm.NtError) as e:
        rocm.lower(bad)
    assert e.value.status == rocm.NT_E_INVALID


def test_malformed_tapes_are_rejected(rocm, tapes):
    flat = tapes["C1"]
    forward_ref = _mutated(flat)
    forward_ref["arg_a"][5] = 20
    with pytest.raises(rocm.NtError) as e:
        rocm.lower(forward_ref)
    assert e.value.status == rocm.NT_E_INVALID
    bad_op = _mutated(flat)
    bad_op["op"][7] = 99
    with pytest.raises(rocm.NtError) as e:
        rocm.lower(bad_op)
    assert e.value.status == rocm.NT_E_INVALID
    bad_input = _mutated(flat, input_node=np.array([0, 1, 2, 3, 5], dtype=np.int32))
    with pytest.raises(rocm.NtError):
        rocm.lower(bad_input)
    with pytest.raises(rocm.NtError) as e:
        rocm.lower(flat, rocm.options(block=100))
    assert e.value.status == rocm.NT_E_INVALID


def test_lower_reports_needed_length(rocm, tapes):
    from nablatensor_amd.rocm import NtOptions, TapeArrays, lib
    arrays = TapeArrays(tapes["C2"])
    t = arrays.struct()
    o = rocm.options()
    n = C.c_int64(0)
    assert lib().nt_lower(C.byref(t), C.byref(o), None, C.byref(n)) == 0
    small = C.create_string_buffer(16)
    m = C.c_int64(16)
    assert lib().nt_lower(C.byref(t), C.byref(o), small, C.byref(m)) == rocm.NT_E_INVALID
    assert m.value == n.value


@pytest.mark.parametrize("name", ["C1", "C2", "C3", "C4", "C5"])
@pytest.mark.parametrize("precision", ["fp64", "fp32"])
def test_offline_gfx950_compile_has_no_scratch(rocm, tapes, name, precision):
    info = rocm.compile_check(tapes[name], rocm.options(precision))
    assert info["scratch_bytes"] == 0
    assert 0 < info["vgprs"] <= 512


def test_one_wave_kernel_near_two_waves_is_compiled_for_two(rocm, tapes):
    """A replay kernel that needs a little more than two waves' 256 VGPRs
    (the 16-asset worst-of in fp64: 270) runs one wave per SIMD; the engine
    compiles it again with launch bounds asking for two and keeps that code,
    which fits without scratch. An explicit waves option is left as asked."""
    info = rocm.compile_check(tapes["C5"], rocm.options("fp64"))
    assert info["scratch_bytes"] == 0 and 0 < info["vgprs"] <= 256, info
    one = rocm.compile_check(tapes["C5"], rocm.options("fp64", waves=1))
    assert one["scratch_bytes"] == 0 and 256 < one["vgprs"] <= 256 + 16, one


def test_spilling_kernel_is_declined(rocm, nt):
    """A kernel that would spill to scratch is declined with NT_E_UNSUPPORTED,
    as the reference's engines decline a tape in compile() (AadEngine.java:50-59),
    unless the caller opts in with allow_spill. The tape: a 96-fixing Asian call
    lowered without its step loop and swept in reverse with every forward
    value kept (checkpoint policy "store all", no segments), so every value
    stays live until the sweep (600 nodes, more than 512 VGPRs hold)."""
    flat = nt.record(nt.Products.asianCall(), nt.EquityMarket.atmOneYear(), nt.TimeGrid.uniform(96)).flat()
    opts = dict(mode=rocm.NT_MODE_REVERSE, roll=-1, checkpoint=rocm.NT_CKPT_STORE_ALL)
    with pytest.raises(rocm.NtError) as e:
        rocm.compile_check(flat, rocm.options("fp64", **opts))
    assert e.value.status == rocm.NT_E_UNSUPPORTED
    assert "declines" in str(e.value) and "spill" in str(e.value) and "allow_spill" in str(e.value)
    info = rocm.compile_check(flat, rocm.options("fp64", allow_spill=True, **opts))
    assert info["scratch_bytes"] > 0 and info["loop_period"] == 0
    # the same tape with its step loop rolled, or cut into checkpointed segments, needs no scratch
    assert rocm.compile_check(flat, rocm.options("fp64", mode=rocm.NT_MODE_REVERSE))["scratch_bytes"] == 0
    info = rocm.compile_check(flat, rocm.options("fp64", mode=rocm.NT_MODE_REVERSE, roll=-1))
    assert info["scratch_bytes"] == 0 and info["n_segments"] == 13 and info["checkpoint"] == rocm.NT_CKPT_RECOMPUTE
