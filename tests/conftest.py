"""Shared fixtures. GPU tests are marked `gpu`; everything else runs on the CPU."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device) and the built libdcn")


@pytest.fixture(scope="session")
def oracle():
    import oracle as _oracle

    _oracle.load()
    return _oracle


@pytest.fixture(scope="session")
def dcn():
    from jasnamacos_amd import deform_conv

    deform_conv.lib()
    return deform_conv


@pytest.fixture(scope="session")
def gpu_ctx(dcn):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible HIP device")
    ctx = dcn.HipDeformConv(0)
    yield ctx
    ctx.close()


def f16(a) -> np.ndarray:
    return np.asarray(a, dtype=np.float32).astype(np.float16)
