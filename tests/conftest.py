"""pytest configuration: the `gpu` marker and import paths.

`-m "not gpu"` runs the CPU suite (oracle pins, host logic, library exports);
`-m gpu` runs the parity tests through the C-ABI on an MI355X.
"""
import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "fastllm-py_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU and the built HIP library")


@pytest.fixture(scope="session")
def torch_gpu():
    """torch with a visible GPU; GPU tests fail (not skip) when the library is missing."""
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm GPU visible")
    from fastllm_py import _native

    _native.load()  # raises FileNotFoundError if the .so was not built
    return torch
