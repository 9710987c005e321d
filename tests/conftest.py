"""Shared pytest configuration: the ``gpu`` marker and common helpers."""

from __future__ import annotations

import os
import sys

import pytest

REPO = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if REPO not in sys.path:
    sys.path.insert(0, REPO)

# North-star tolerance on bf16 outputs against the fp32 oracle.
MAX_ABS_TOL = 2e-2
MEAN_ABS_TOL = 2e-3


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs through libmxattn.so)")


def gpu_available() -> bool:
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def pytest_collection_modifyitems(config, items):
    if gpu_available():
        return
    skip = pytest.mark.skip(reason="no GPU in this environment")
    for item in items:
        if "gpu" in item.keywords:
            item.add_marker(skip)


def assert_close_to_oracle(out, ref, label=""):
    """max-abs <= 2e-2 and mean-abs <= 2e-3 of bf16 output against the fp32 oracle."""
    import torch
    diff = (out.float().cpu() - ref.float().cpu()).abs()
    assert torch.isfinite(out.float()).all(), f"{label}: non-finite output"
    max_abs = diff.max().item()
    mean_abs = diff.mean().item()
    assert max_abs <= MAX_ABS_TOL, f"{label}: max-abs {max_abs:.3e} > {MAX_ABS_TOL}"
    assert mean_abs <= MEAN_ABS_TOL, f"{label}: mean-abs {mean_abs:.3e} > {MEAN_ABS_TOL}"
    return max_abs, mean_abs
