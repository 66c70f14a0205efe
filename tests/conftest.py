"""Shared test setup. `gpu` tests need a HIP device (MI355X) and the built
libholo_hip.so; everything else runs on the CPU against the oracle."""
import os
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parent.parent
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and libholo_hip.so")


def splitmix64(x: np.ndarray) -> np.ndarray:
    """splitmix64 finalizer over a uint64 array (the seeded generator of the configs)."""
    x = (x + np.uint64(0x9E3779B97F4A7C15)).astype(np.uint64)
    x = (x ^ (x >> np.uint64(30))) * np.uint64(0xBF58476D1CE4E5B9)
    x = (x ^ (x >> np.uint64(27))) * np.uint64(0x94D049BB133111EB)
    return x ^ (x >> np.uint64(31))


def u16_patterns(n: int, seed: int) -> np.ndarray:
    """x[i] = splitmix64(seed ^ i) >> 48: uniform over all 65536 bit patterns."""
    with np.errstate(over="ignore"):
        idx = np.arange(n, dtype=np.uint64) ^ np.uint64(seed)
        return (splitmix64(idx) >> np.uint64(48)).astype(np.uint16)


@pytest.fixture(scope="session")
def torch_cuda():
    import torch
    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    return torch


@pytest.fixture(scope="session")
def backend(torch_cuda):
    from hologram_amd import HipBackend
    be = HipBackend(device=0, stream=torch_cuda.cuda.current_stream().cuda_stream)
    yield be
    be.synchronize()
    be.close()


def to_dev(torch, arr: np.ndarray):
    """Copy a numpy array to a device tensor of the same bytes (uint8 view)."""
    t = torch.from_numpy(np.ascontiguousarray(arr).view(np.uint8).reshape(-1).copy())
    return t.to("cuda")


def from_dev(t, dtype, count=None) -> np.ndarray:
    out = t.cpu().numpy().view(dtype)
    return out if count is None else out[:count]
