"""Shared pytest setup: markers, import paths and build-on-demand of the
checker (oracle) and the HIP library when nothing is built yet."""
import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
for path in (REPO, os.path.join(REPO, "src")):
    if path not in sys.path:
        sys.path.insert(0, path)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


@pytest.fixture(scope="session")
def oracle():
    from oracle import gru_oracle

    gru_oracle.build()
    return gru_oracle


@pytest.fixture(scope="session")
def hip_lib():
    from rnn_kernel_amd import _lib

    if not os.path.exists(_lib.LIB_PATH):
        from rnn_kernel_amd import build as rka_build

        rka_build.build()
    return _lib.load()


@pytest.fixture(scope="session")
def gpu(hip_lib):
    import torch

    if not torch.cuda.is_available():
        pytest.fail("gpu-marked test run without a visible GPU")
    if not hip_lib.rka_device_supported(torch.cuda.current_device()):
        pytest.fail("GPU is not gfx950: " + hip_lib.rka_last_error().decode())
    return torch.device("cuda", torch.cuda.current_device())
