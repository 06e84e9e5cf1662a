"""Shared test setup.

Markers: `gpu` tests need an MI355X and the built libbwpp_hip; everything
else runs on the CPU (the oracle, host logic, the C ABI without compute).
"""
from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "bluewolf-plus-plus_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden", "ref_vectors.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built libbwpp_hip")


@pytest.fixture(scope="session")
def oracle():
    from oracle.oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.oracle import RefLib
    if not RefLib.available():
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    return RefLib()


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def be():
    """libbwpp_hip handle on cuda:0, launching on torch's current stream."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test without a visible GPU")
    import bwpp
    backend = bwpp.HipBackend(0)
    backend.set_stream(torch.cuda.current_stream())
    yield backend
    backend.close()


def assert_bits_equal(a, b, what=""):
    """Bitwise float32 equality; NaNs must coincide (payloads not compared)."""
    a = np.asarray(a, dtype=np.float32)
    b = np.asarray(b, dtype=np.float32)
    assert a.shape == b.shape, (what, a.shape, b.shape)
    na, nb = np.isnan(a), np.isnan(b)
    assert np.array_equal(na, nb), f"{what}: NaN positions differ"
    ua = a.view(np.uint32)[~na]
    ub = b.view(np.uint32)[~nb]
    bad = np.nonzero(ua != ub)[0]
    assert bad.size == 0, f"{what}: {bad.size} elements differ, first at flat {bad[:5]}"


def rel_max_err(got, want):
    """max|got - want| / max|want| over finite reference entries."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    fin = np.isfinite(want)
    denom = np.max(np.abs(want[fin])) if fin.any() else 1.0
    if denom == 0:
        denom = 1.0
    return float(np.max(np.abs(got[fin] - want[fin])) / denom) if fin.any() else 0.0
