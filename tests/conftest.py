"""Test configuration.

Markers:
  gpu  needs an MI355X (gfx950) and the built libeakv.so; run with -m gpu.
Everything unmarked runs on a CPU-only machine against the oracle, the host
logic and the exported C ABI.
"""
import os
import sys
import zlib

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for p in (ROOT, os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a gfx950 GPU and libeakv.so")


@pytest.fixture
def rng(request):
    seed = zlib.crc32(request.node.nodeid.encode())
    return np.random.default_rng(seed)


def tol_close(got, want, atol=1e-4, rtol=1e-5):
    """The parity bar for floating-point results: |got-want| <= atol + rtol*|want|."""
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want)
    lim = atol + rtol * np.abs(want)
    bad = ~(err <= lim)
    return (not bad.any()), float(err.max(initial=0.0)), int(bad.sum())
