"""Shared pytest setup.

`gpu`-marked tests need an MI355X (ROCm device) and the in-tree
libntlowbit.so; everything else runs on the CPU.  The product package lives in
nano-train_amd/ (a directory name that is not importable), so its parent is
put on sys.path here, next to the repo root for `oracle`.
"""

from __future__ import annotations

import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG_PARENT = os.path.join(ROOT, "nano-train_amd")
for p in (ROOT, PKG_PARENT):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


@pytest.fixture(scope="session")
def gpu_device():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no ROCm device visible")
    return torch.device("cuda", 0)
