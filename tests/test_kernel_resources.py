"""The compiled kernels' register and scratch use, from the compiler's
resource remarks that the build records (novann_amd/_build/kernel_resources.json).

A device function the compiler did not inline shows up under its own name; a
per-band function of the band convolution that was outlined once carried its
workgroup barriers into a called function, spilled 448 bytes per lane and
hung its epilogue test.  So: nothing outlined, no vector-register spills,
and the band convolution keeps four workgroups per CU (the occupancy its
schedule relies on: each workgroup's loads, products and stores overlap those
of the others).  CPU-only: it reads what the build wrote."""
import json
import os

import pytest

RES = os.path.join(os.path.dirname(__file__), "..", "novann_amd", "_build", "kernel_resources.json")


@pytest.fixture(scope="module")
def res():
    if not os.path.exists(RES):
        pytest.skip("library not built here (run __graft_entry__.build())")
    with open(RES) as f:
        return json.load(f)


def test_every_function_is_a_kernel(res):
    # function-local entities (lambdas' call operators) mangle as _ZZ...
    outlined = [n for n in res if n.startswith("_ZZ")]
    assert not outlined, outlined[:5]


def test_no_vector_register_spills(res):
    spilled = {n: r for n, r in res.items() if r.get("vgpr_spill", 0)}
    assert not spilled, list(spilled)[:5]


def test_scratch_only_where_expected(res):
    # one kernel uses scratch by design, nothing else: the guarded edge-tile
    # Linear kernel (one workgroup per CU, 110 KB of LDS) spills 14 scalar
    # registers
    for name, r in res.items():
        if not r.get("scratch", 0):
            continue
        assert "linear_kernel" in name and r.get("vgpr_spill", 0) == 0, (name, r)


def test_band_convolution_keeps_four_workgroups_per_cu(res):
    band = {n: r for n, r in res.items() if "conv2d_band_kernel" in n}
    assert band
    for name, r in band.items():
        assert r["occupancy"] >= 4 and r.get("scratch", 0) == 0, (name, r)
