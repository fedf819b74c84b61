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


def copy_model_to_oracle(orc_mod, g, cfg, seed=0):
    """An oracle model holding the device model's packed bytes (copied back
    with wst_memcpy_d2h), for full-size shapes where the host quantiser would
    take minutes. The device packer is byte-equal to the host quantiser
    (tests/test_gpu_fixture_fused.py), so this is the same model either way."""
    from whetstone_amd import ffi
    o = orc_mod.Model(cfg, seed, pack=False)
    names = ["embed"] + ([] if cfg["tied"] else ["lm_head"])
    names += [f"L{l}.{t}" for l in range(cfg["n_layers"]) for t in ("qkv", "o", "gate_up", "down")]
    for name in names:
        qw, si, sb, i, n = g.tensor(name)
        p = o.tensor(name)
        assert (p.in_f, p.out_f) == (i, n), name
        for dst, src in ((p.qw, qw), (p.si, si), (p.sb, sb)):
            ffi.check(ffi.lib().wst_memcpy_d2h(dst.ctypes.data, src, dst.nbytes))
    return o


def assert_streams(got, want, margins, tie_margin=1e-4):
    """Identical, or the first divergence sits on a near-tie of the oracle
    (top-2 margin below tie_margin), where f32 rounding legitimately decides.
    Returns the number of leading tokens that agree."""
    got, want = list(map(int, got)), list(map(int, want))
    assert len(got) == len(want), (len(got), len(want))
    if got == want:
        return len(got)
    k = next(i for i, (a, b) in enumerate(zip(got, want)) if a != b)
    assert margins[k] < tie_margin, f"diverged at step {k}: {got[k]} vs {want[k]}, margin {margins[k]}"
    return k


def ns_tol(logits) -> float:
    """The north star's logit tolerance as one number for a vector: 1e-2
    max-abs plus 1e-3 of its largest magnitude. Two implementations within
    it of each other can pick different greedy tokens only where a top-2
    margin is below twice it. (Twice the measured distance between two
    vectors bounds their own argmax flip by construction, so it tests
    nothing; this bound is fixed before the run.)"""
    return 1e-2 + 1e-3 * float(np.max(np.abs(np.asarray(logits, np.float64))))
