"""Test setup: registers the ``gpu`` marker and imports the package under the
name ``light_vllm_amd`` (the directory ``light-vllm_amd`` is not an identifier)."""

from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))
importlib.import_module("light-vllm_amd")


def pytest_configure(config: pytest.Config) -> None:
    config.addinivalue_line("markers", "gpu: runs HIP kernels on an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    import torch

    return torch.cuda.is_available()
