import os
import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "vllm-exl3_amd", ROOT / "oracle", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libexl3_mi355x.so)")


@pytest.fixture(scope="session")
def gpu():
    """The HIP device; GPU tests skip without one and fail if the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no HIP device")
    from vllm_exl3_amd import _lib

    _lib.load()  # raises when the library is not built
    return torch.device("cuda", 0)


@pytest.fixture(params=["auto", "persistent"])
def gemv_policy(request, monkeypatch):
    """Decode GEMV kernel choice for the test: the cost model's ("auto"), or
    the persistent kernel forced (EXL3_GEMV_KERNEL, read by the library's
    planner on every call), so both kernels are checked on the same inputs."""
    monkeypatch.setenv("EXL3_GEMV_KERNEL", request.param)
    return request.param
