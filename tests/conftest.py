"""pytest configuration: the `gpu` marker, import paths and shared fixtures.

Tests marked `gpu` need an MI355X and run the HIP library; every other test
runs on the CPU (oracle, comparators, C-ABI validation, weight files).
"""

from __future__ import annotations

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (ROOT, os.path.join(ROOT, "cu-vit_amd"), os.path.join(ROOT, "oracle"),
             os.path.join(ROOT, "tests")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X GPU and the built HIP library")


@pytest.fixture(scope="session")
def oracle():
    from oracle import Oracle

    return Oracle()


@pytest.fixture(scope="session")
def reference():
    from oracle import Reference, reference_available

    if not reference_available():
        pytest.skip("oracle/_ref (the reference's CPU code) is not built on this host")
    return Reference()


@pytest.fixture(scope="session")
def reference_or_none():
    """The reference's CPU code where oracle/_ref is built, else None (for
    tests whose extra reference check is optional)."""
    from oracle import Reference, reference_available

    return Reference() if reference_available() else None


@pytest.fixture(scope="session")
def lib():
    import cuvit_amd

    return cuvit_amd.library()


@pytest.fixture(scope="session")
def cuvit():
    import cuvit_amd

    cuvit_amd.library()
    return cuvit_amd


@pytest.fixture(scope="session")
def device():
    """cuda:0 for GPU tests. On a GPU host a missing device is a failure, not a skip."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test collected but no GPU is visible")
    return torch.device("cuda:0")


def to_device(array: np.ndarray, device):
    import torch

    return torch.from_numpy(np.ascontiguousarray(array)).to(device)


def to_host(tensor) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return tensor.detach().cpu().numpy()


def bf16_tensor(bits: np.ndarray, device):
    """A torch bfloat16 tensor holding the given bf16 bit patterns."""
    import torch

    return torch.from_numpy(np.ascontiguousarray(bits, dtype=np.uint16).view(np.int16)).to(
        device).view(torch.bfloat16)


def bf16_bits(tensor) -> np.ndarray:
    import torch

    torch.cuda.synchronize()
    return tensor.detach().view(torch.int16).cpu().numpy().view(np.uint16)
