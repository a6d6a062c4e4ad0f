"""Shared fixtures for the parity suite.

Markers: ``gpu`` -- needs an MI355X (runs the HIP path through the C ABI).
Everything unmarked runs on the CPU: the oracle against golden vectors /
closed forms, host logic, and the C-ABI library's exported symbols.
"""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X); runs the HIP kernels")


def rel_frob(got, want):
    """Relative Frobenius error ||got - want|| / ||want||, accumulated in f64."""
    got = np.asarray(got, np.float64).ravel()
    want = np.asarray(want, np.float64).ravel()
    den = np.linalg.norm(want)
    num = np.linalg.norm(got - want)
    return num / den if den > 0 else num


# Parity tolerance for fp32 results computed in a different summation order
# than the reference CPU path (1e-5 relative Frobenius).
TOL = 1e-5


@pytest.fixture(scope="session")
def orc():
    from oracle import pyorc
    pyorc.build()
    return pyorc


@pytest.fixture(scope="session")
def rnn():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    import rustnn_amd
    rustnn_amd.lib()
    return rustnn_amd


def to_dev(a):
    import torch
    return torch.from_numpy(np.ascontiguousarray(a)).cuda()


def to_host(t):
    import torch
    torch.cuda.synchronize()
    return t.detach().cpu().numpy()
