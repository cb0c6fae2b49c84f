import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libqasr_hip.so)")
    config.addinivalue_line("markers", "slow: long-running CPU case")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle
    oracle.lib()
    oracle.set_threads(min(8, os.cpu_count() or 8))
    return oracle


@pytest.fixture(scope="session")
def dev():
    """The GPU handle; GPU tests fail (not skip) when the HIP library or device is missing."""
    from qwenasr_amd import Device, device_count
    assert device_count() >= 1, "no HIP device visible"
    d = Device(0)
    yield d
    d.close()


def rng(seed):
    return np.random.default_rng(seed)


def bf16(a):
    from qwenasr_amd.synth import f32_to_bf16
    return f32_to_bf16(np.asarray(a, np.float32))


def bf16f(a):
    return (np.asarray(a, np.uint16).astype(np.uint32) << 16).view(np.float32)
