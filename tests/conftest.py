"""Shared fixtures for the parity suite.

Markers: ``gpu`` tests need an MI355X (gfx950) and the built libclove_hip.so;
everything else runs on the CPU.  Inputs are generated with numpy's PCG64
from fixed seeds (Clove's own RNG is unseeded, backend.rs:965-974), and the
same bytes go to the HIP backend and to the CPU oracle.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X and the built HIP library")


@pytest.fixture(scope="session")
def hip():
    """Initialises the HIP backend once per session; the device must work."""
    import clove_amd

    clove_amd.init(0)
    yield clove_amd
    clove_amd.synchronize()


def rng(seed: int) -> np.random.Generator:
    return np.random.Generator(np.random.PCG64(seed))


def assert_close(got, want, rtol, atol, what=""):
    """|got - want| <= atol + rtol * |want| elementwise, with a report of the
    worst element on failure."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    err = np.abs(got - want)
    bound = atol + rtol * np.abs(want)
    bad = ~(err <= bound)
    if bad.any():
        i = np.unravel_index(np.argmax(np.where(bad, err - bound, -np.inf)), err.shape)
        raise AssertionError(
            f"{what}: {int(bad.sum())} of {err.size} elements out of tolerance "
            f"(rtol={rtol}, atol={atol}); worst at {i}: got {got[i]!r} want {want[i]!r}, "
            f"max abs err {err.max():.3e}")
