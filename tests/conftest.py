# SPDX-License-Identifier: Apache-2.0
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("oracle", "kimi-k3-in-c_amd", os.path.join("tests", "golden")):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libk3amd.so)")


@pytest.fixture(scope="session")
def k3():
    import k3amd
    k3amd.lib()
    return k3amd


@pytest.fixture(scope="session")
def wl():
    import workloads
    return workloads


@pytest.fixture(scope="session")
def orc():
    from oracle import Oracle
    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle import Ref
    if not Ref.available():
        pytest.skip("oracle/_ref not built (needs the reference sources at build time)")
    return Ref()


@pytest.fixture(scope="session")
def fx():
    return dict(np.load(os.path.join(ROOT, "tests", "golden", "ref_fixtures.npz")))


@pytest.fixture(scope="session")
def gold():
    return dict(np.load(os.path.join(ROOT, "tests", "golden", "ref_golden.npz")))


@pytest.fixture(scope="session")
def gpu(k3):
    """The device path. Fails (never skips) when no device is usable: a GPU test that
    silently did not run would read as a pass."""
    rc = k3.lib().k3d_init()
    if rc != 0:
        pytest.fail("no usable HIP device: " + k3.lib().k3d_error().decode())
    return k3


def max_err_rel_inf(got, ref):
    """max|got - ref| / ||ref||inf, the tolerance measure of the fp32 GEMV paths."""
    got = np.asarray(got, np.float64)
    ref = np.asarray(ref, np.float64)
    scale = np.abs(ref).max()
    return float(np.abs(got - ref).max() / (scale if scale > 0 else 1.0))
