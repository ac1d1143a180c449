import os
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")
FIXTURE_SMTX = os.path.join(GOLDEN, "body_decoder_layer_2_ffn_conv1.smtx")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


@pytest.fixture(scope="session")
def fixture_text():
    with open(FIXTURE_SMTX) as f:
        return f.read()


@pytest.fixture(scope="session")
def torch_cuda():
    """torch with a visible GPU, for device buffers of the GPU tests."""
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch


def exact_values(rng, n):
    """Values in {+-1, +-1/2, +-2}: products with k/256 are exact in fp16/fp32."""
    return rng.choice(np.array([-2.0, -1.0, -0.5, 0.5, 1.0, 2.0], np.float32), size=n)


def exact_dense(rng, shape):
    """Values k/256 with |k| <= 256 (exact in fp16, bf16 needs |k| <= 256 too)."""
    return (rng.integers(-256, 257, size=shape) / 256.0).astype(np.float32)
