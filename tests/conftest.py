"""Shared test plumbing.

Markers: ``gpu`` tests need a real MI355X (they call the HIP library through
its C ABI); everything else runs on the CPU.  The oracle (oracle/) is the
checker in both.
"""
from __future__ import annotations

import importlib
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an AMD gfx950 GPU and the built HIP library")


@pytest.fixture(scope="session")
def orc():
    from oracle.oracle import oracle
    return oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.oracle import reference
    r = reference()
    if r is None:
        pytest.skip("reference kernel library not buildable here (no /root/reference)")
    return r


@pytest.fixture(scope="session")
def hip():
    """The HIP binding; a missing library is an error, never a skip."""
    return importlib.import_module("see-ai_amd.hip")


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("gpu test run without a visible GPU")
    return torch


def maxrel(a, b) -> float:
    """max|a-b| / max|b| per tensor (tool/frontier_exec.py:54's convention)."""
    a = np.asarray(a, np.float64)
    b = np.asarray(b, np.float64)
    if a.size == 0:
        return 0.0
    den = np.max(np.abs(b))
    num = np.max(np.abs(a - b))
    if den == 0.0:
        return float(num)
    return float(num / den)


def bits_equal(a, b) -> bool:
    a = np.ascontiguousarray(a)
    b = np.ascontiguousarray(b)
    if a.dtype == np.float32:
        return np.array_equal(a.view(np.uint32), b.view(np.uint32))
    return np.array_equal(a, b)
