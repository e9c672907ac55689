"""Shared test configuration: import paths, the `gpu` marker and small helpers."""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
for p in (REPO, REPO / "int8-kvcache_amd"):
    if str(p) not in sys.path:
        sys.path.insert(0, str(p))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def bf16_to_f32(t: torch.Tensor) -> np.ndarray:
    """Exact float32 numpy copy of a (CPU or GPU) tensor."""
    return t.detach().to("cpu", torch.float32).numpy()


def metrics(out: np.ndarray, ref: np.ndarray):
    """(max |diff|, cosine, relative L2) of two arrays, computed in float64."""
    a = np.asarray(out, np.float64).reshape(-1)
    b = np.asarray(ref, np.float64).reshape(-1)
    diff = np.abs(a - b).max() if a.size else 0.0
    cos = float(a @ b / (np.linalg.norm(a) * np.linalg.norm(b) + 1e-30))
    rel = float(np.linalg.norm(a - b) / (np.linalg.norm(b) + 1e-30))
    return float(diff), cos, rel


# Parity bar for attention outputs against the fp32 oracle (the project's acceptance bar).
MAX_ABS = 2e-2
MIN_COS = 0.9999


@pytest.fixture(scope="session")
def cuda():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda:0")
