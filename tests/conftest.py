"""Shared test setup.

Markers: `gpu` tests need an MI355X (HIP device) and the built
libwhetstone_hip.so; everything else runs on the CPU.
"""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a HIP GPU (MI355X) and the built library")


@pytest.fixture(scope="session")
def orc():
    from oracle import oracle as O
    O.lib()
    return O


@pytest.fixture(scope="session")
def wk():
    """The product library; gpu tests only. Fails loudly if it is not built."""
    from whetstone_amd import kernels
    n = kernels.device_count()
    if n < 1:
        pytest.fail("no HIP device visible to a gpu-marked test")
    return kernels


def f16(orc_mod, x):
    """f32 values -> f16 bit patterns (np.uint16) via the oracle's RNE."""
    return orc_mod.f16_bits(np.asarray(x, np.float32))


def dev_f16(wk_mod, bits):
    """Upload f16 bit patterns as a float16 device buffer (no numeric conversion)."""
    return wk_mod.DeviceBuffer.from_array(np.ascontiguousarray(bits, np.uint16).view(np.float16))
