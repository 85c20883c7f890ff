import os
import sys

import numpy as np
import pytest

# torch (device buffers in the GPU tests) bundles its own HIP runtime; it must
# be loaded before libmemvanta_hip.so so that both resolve to one runtime.
# Imported here, it is, however the tests are selected.
try:
    import torch  # noqa: F401
except ImportError:
    torch = None

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device 0)")
    config.addinivalue_line("markers", "slow: long CPU test")


@pytest.fixture(scope="session")
def oracle():
    from oracle.pyoracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def ref():
    from oracle.pyoracle import Ref, ref_available

    if not ref_available():
        pytest.skip("compiled reference (oracle/_ref) not built here")
    return Ref()


@pytest.fixture(scope="session")
def ctx():
    from memvanta_amd import capi

    c = capi.Context(0)
    yield c
    c.close()


def golden(name):
    path = os.path.join(GOLDEN, name)
    return np.load(path, allow_pickle=False)


def bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def assert_bitexact(got, want, what=""):
    got = np.ascontiguousarray(got, np.float32)
    want = np.ascontiguousarray(want, np.float32)
    assert got.shape == want.shape, (got.shape, want.shape)
    bad = np.flatnonzero(bits(got) != bits(want))
    if bad.size:
        i = bad[0]
        raise AssertionError(f"{what}: {bad.size}/{got.size} elements differ; first at {i}: "
                             f"{got.ravel()[i]!r} vs {want.ravel()[i]!r}; max |diff| {np.abs(got - want).max()}")
