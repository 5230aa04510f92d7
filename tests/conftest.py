"""Shared test setup: the `gpu` marker, import paths and small helpers."""
import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels through the C ABI)")


def gpu_available() -> bool:
    try:
        import ctypes
        hip = ctypes.CDLL("libamdhip64.so")
        n = ctypes.c_int(0)
        return hip.hipGetDeviceCount(ctypes.byref(n)) == 0 and n.value > 0
    except OSError:
        return False


@pytest.fixture(scope="session")
def ctx():
    """One library context on device 0 for the whole GPU session."""
    import rce_amd
    c = rce_amd.Context(0)
    yield c
    c.close()


def lcg_uniform(seed: int, n: int, a: float) -> np.ndarray:
    """The reference tests' Lcg (spec/checker/tests/support/toy_gpt2.rs L18-27;
    kquant.rs tests L401-409): uniform in [-a, a) from a fixed 64-bit LCG."""
    out = np.empty(n, np.float32)
    s = seed & 0xFFFFFFFFFFFFFFFF
    for i in range(n):
        s = (s * 6364136223846793005 + 1442695040888963407) & 0xFFFFFFFFFFFFFFFF
        v = np.float32(s >> 40) / np.float32(1 << 24) * np.float32(2.0) - np.float32(1.0)
        out[i] = np.float32(v) * np.float32(a)
    return out


def normal_weights(rng: np.random.Generator, shape, sigma: float) -> np.ndarray:
    return (rng.standard_normal(shape) * sigma).astype(np.float32)
