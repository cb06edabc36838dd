"""Shared test setup: the `gpu` marker, import paths for the product's ctypes binding
(julia-cuda_amd/julia_hip.py) and the CPU oracle (oracle/oracle.py), and device helpers."""

import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for sub in ("julia-cuda_amd", "oracle"):
    p = os.path.join(ROOT, sub)
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def torch_cuda():
    """torch with a GPU; the GPU tests need it for device memory and streams."""
    import torch

    if not torch.cuda.is_available():
        pytest.fail("the gpu tests need a GPU (torch.cuda.is_available() is False)")
    return torch


def to_dev(torch, a):
    """numpy array -> device tensor (f16 bit patterns as float16)."""
    a = np.ascontiguousarray(a)
    if a.dtype == np.uint16:
        return torch.from_numpy(a.view(np.float16)).cuda()
    return torch.from_numpy(a).cuda()


def f16_bits(t):
    """device float16 tensor -> numpy uint16 bit patterns."""
    return t.detach().cpu().numpy().view(np.uint16)
