"""Test configuration: import paths and the ``gpu`` marker.

CPU tests (``-m "not gpu"``) cover the oracle against its pins, the host-side
logic (validation, dispatch plans, C-ABI argument checks) and that the HIP
library loads and exports every symbol of include/switchyard.h. GPU tests
(``-m gpu``) call the HIP kernels through the C ABI and compare them with the
oracle.
"""

from __future__ import annotations

import pathlib
import sys

import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
for p in (ROOT / "blackwell-switchyard_amd", ROOT):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs on the GPU box")
    config.addinivalue_line("markers", "slow: long-running")


def has_gpu() -> bool:
    import torch

    return torch.cuda.is_available()
