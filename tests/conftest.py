"""Shared test setup.

`gpu`-marked tests need a real MI355X and run on the GPU box
(`pytest -m gpu`); everything else runs on the CPU (`pytest -m "not gpu"`).
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden", "qwen35_vision_tiny.npz")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (run with -m gpu on the GPU box)")


@pytest.fixture(scope="session")
def golden():
    import numpy as np

    return np.load(GOLDEN)


@pytest.fixture(scope="session")
def torch_gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.fail("a gpu-marked test ran without a visible GPU")
    return torch
