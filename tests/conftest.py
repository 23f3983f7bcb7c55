"""Shared pytest configuration.

Markers:
  gpu -- needs an MI355X (gfx950) and the built libqasr_hip.so; these are the
         parity tests proper and run on a GPU. Everything else runs on CPU.
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))

GOLDEN = ROOT / "tests" / "golden" / "golden.npz"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def golden():
    with np.load(GOLDEN, allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


@pytest.fixture(scope="session")
def dev():
    """The GPU device. Fails (does not skip) when no GPU is visible: gpu tests
    are only selected where one is expected."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu test selected but torch.cuda.is_available() is False")
    from qwenasr_amd import _lib

    _lib.lib()  # raises QasrLibraryMissing if the HIP library is not built
    return torch.device("cuda:0")


def assert_close(got, ref, rtol, atol, what=""):
    """|got - ref| <= atol + rtol * |ref| elementwise (NaN must match NaN)."""
    got = np.asarray(got, dtype=np.float64)
    ref = np.asarray(ref, dtype=np.float64)
    assert got.shape == ref.shape, f"{what}: shape {got.shape} != {ref.shape}"
    nan_g, nan_r = np.isnan(got), np.isnan(ref)
    assert np.array_equal(nan_g, nan_r), f"{what}: NaN pattern differs"
    g, r = got[~nan_g], ref[~nan_r]
    err = np.abs(g - r)
    bound = atol + rtol * np.abs(r)
    bad = err > bound
    if bad.any():
        i = int(np.argmax(err - bound))
        raise AssertionError(
            f"{what}: {int(bad.sum())}/{g.size} elements out of tolerance "
            f"(rtol={rtol}, atol={atol}); worst at {i}: got {g[i]!r} ref {r[i]!r} err {err[i]:.3e}")
