"""Shared fixtures.  `-m gpu` tests run the HIP library on a GPU and check it
against the CPU oracle; the rest run anywhere."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.abspath(os.path.join(os.path.dirname(__file__), ".."))
sys.path.insert(0, os.path.join(ROOT, "minicpm5.cpp_amd", "python"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
GOLDEN = os.path.join(ROOT, "tests", "golden")

import mcpm  # noqa: E402
import oracle as O  # noqa: E402


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library)")


@pytest.fixture(scope="session")
def orc():
    return O.oracle()


@pytest.fixture(scope="session")
def ref():
    r = O.reference()
    if r is None:
        pytest.skip("oracle/_ref (the reference's compiled ops) not built here")
    r.ref_set_threads(8)
    return r


@pytest.fixture(scope="session")
def lib():
    return mcpm.load_library()


@pytest.fixture(scope="session")
def ctx():
    c = mcpm.Context(0)
    yield c
    c.close()


# Host arrays whose address is passed to C stay referenced until the test ends:
# P(x.copy()) would otherwise hand C the address of an already-freed temporary.
_HOLD = []


@pytest.fixture(autouse=True)
def _hold_host_arrays():
    yield
    _HOLD.clear()


def P(a):
    _HOLD.append(a)
    return a.ctypes.data


def golden(name):
    return np.load(os.path.join(GOLDEN, name))


def announce(msg):
    """Names the GPU case about to run, flushed, so a fault points at it."""
    print(f"[case] {msg}", flush=True)


def rel_err(a, b):
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    return float(np.abs(a - b).max() / max(np.abs(b).max(), 1e-30))


def assert_close(a, b, tol=1e-3, floor=1e-2):
    """Per-op parity metric: normwise max relative error, and per element
    |a-b| <= tol*max(|b_i|, floor*max|b|)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    assert a.shape == b.shape
    scale = np.abs(b).max()
    assert rel_err(a, b) <= tol, f"normwise rel err {rel_err(a, b)} > {tol}"
    bound = tol * np.maximum(np.abs(b), floor * scale)
    bad = np.abs(a - b) > bound
    assert not bad.any(), f"{bad.sum()} elements outside the per-element bound"


def assert_bits(a, b):
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    assert a.shape == b.shape, (a.shape, b.shape)
    av, bv = a.view(np.uint8), b.view(np.uint8)
    if not np.array_equal(av, bv):
        if a.dtype == np.float32:
            diff = np.nonzero(a.view(np.uint32) != b.view(np.uint32))[0]
            i = diff[0]
            raise AssertionError(f"{diff.size} of {a.size} differ; first at {i}: {a.flat[i]!r} vs {b.flat[i]!r}")
        raise AssertionError(f"{np.count_nonzero(av != bv)} bytes differ")
