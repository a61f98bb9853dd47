"""The benchmark workloads at their full dispatch sizes on MI355X, through
properties that hold at any size (the oracle finishes these sizes only in
minutes, so it checks the same kernels at smaller sizes in test_gpu_parity):

* the reference's own aggregates for the Asian call at 2,000,000 scenarios
  (docs/compare/vs-bump-and-revalue.md:39, docs/examples/asian-greeks.md:43-46);
* a dispatch split into two path ranges sums to the whole (exactly up to the
  fp64 summation order), which pins the counter keying at every path index;
* the two derivative modes (reverse sweep and tangent) agree on every sum;
* fp32 reconciles with the fp64 kernel within 1e-5 relative on the price and
  on every Greek (conftest.reconcile);
* the same dispatch twice gives the same bits;
* path offsets near 2^64 wrap exactly as the oracle's.
"""
from __future__ import annotations

import numpy as np
import pytest

import oracle
from conftest import reconcile, reference_values, rel_err

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def rocm():
    from nablatensor_amd import rocm as r
    assert r.probe() > 0, "no gfx950 device visible to libnt_rocm.so"
    return r


def replay(rocm, flat, paths, offset=0, seed=42, **opts):
    with rocm.Executable(flat, rocm.options(**opts)) as x:
        sums, _ = x.replay(paths, offset, seed)
    return sums


def test_asian_2m_reference_aggregates(rocm, tapes):
    ref = reference_values()["asian_call_252_atm_1y_fp64_seed42"]["scenarios_2000000"]
    sums = replay(rocm, tapes["C2"], 2_000_000, precision="fp64")
    r = oracle.to_result(sums, 2_000_000)
    got = {"price": r["price"], "spot": r["gradient"][0], "vol": r["gradient"][2], "rate": r["gradient"][3]}
    for k, v in got.items():
        assert abs(v - ref[k]) <= ref["abs_precision"], (k, v, ref[k])


@pytest.mark.parametrize("name,paths,precision,seed", [("C2", 2_000_000, "fp64", 42),
                                                         ("C3", 20_000_000, "fp32", 42),
                                                         ("C4", 10_000_000, "fp64", 7),
                                                         ("C5", 1_000_000, "fp32", 42)])
def test_split_dispatch_is_additive_and_repeatable(rocm, tapes, name, paths, precision, seed):
    flat = tapes[name]
    cut = (paths * 3) // 5 + 17
    with rocm.Executable(flat, rocm.options(precision)) as x:
        whole, _ = x.replay(paths, 0, seed)
        again, _ = x.replay(paths, 0, seed)
        first, _ = x.replay(cut, 0, seed)
        second, _ = x.replay(paths - cut, cut, seed)
    assert np.array_equal(whole, again)
    assert rel_err(first + second, whole, floor=1e-300) <= 1e-11


@pytest.mark.parametrize("name,paths,seed", [("C2", 2_000_000, 42), ("C3", 20_000_000, 42),
                                             ("C4", 10_000_000, 7)])
def test_tangent_and_reverse_agree_at_full_size(rocm, tapes, name, paths, seed):
    tan = replay(rocm, tapes[name], paths, seed=seed, precision="fp64", mode=rocm.NT_MODE_TANGENT)
    rev = replay(rocm, tapes[name], paths, seed=seed, precision="fp64", mode=rocm.NT_MODE_REVERSE)
    assert rel_err(tan, rev, floor=1e-300) <= 1e-10


@pytest.mark.parametrize("name,paths,seed", [("C3", 20_000_000, 42), ("C5", 1_000_000, 42)])
def test_fp32_reconciles_with_fp64_at_full_size(rocm, tapes, name, paths, seed):
    s32 = replay(rocm, tapes[name], paths, seed=seed, precision="fp32")
    s64 = replay(rocm, tapes[name], paths, seed=seed, precision="fp64")
    errs = reconcile(s32, s64, paths, tapes[name], seed)
    print(name, errs)
    assert errs["ok"], errs


def test_offsets_near_two_to_the_64_wrap_like_the_oracle(rocm, tapes):
    offset = 2**64 - 1500
    sums = replay(rocm, tapes["C2"], 4000, offset=offset, seed=0xFEDCBA9876543210, precision="fp64")
    ref = oracle.replay_sums(tapes["C2"], 4000, offset, 0xFEDCBA9876543210)
    assert rel_err(sums, ref, floor=1e-300) <= 1e-10
