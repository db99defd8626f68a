"""Shared pytest setup: the `gpu` marker, import helpers, common fixtures."""
from __future__ import annotations

import importlib
import sys
from pathlib import Path

import pytest

REPO = Path(__file__).resolve().parents[1]
if str(REPO) not in sys.path:
    sys.path.insert(0, str(REPO))

PKG_NAME = "1188b-reference-kernels_amd"


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP kernels)")


def load_pkg():
    return importlib.import_module(PKG_NAME)


@pytest.fixture(scope="session")
def pkg():
    return load_pkg()


@pytest.fixture(scope="session")
def dev():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU visible")
    return torch.device("cuda:0")


def bits(t):
    """Raw bit pattern of a tensor (int16 view for bf16, int32 for fp32) on the CPU."""
    import torch

    t = t.detach().cpu().contiguous()
    if t.dtype == torch.bfloat16:
        return t.view(torch.int16)
    if t.dtype == torch.float32:
        return t.view(torch.int32)
    return t


def assert_bits_equal(got, ref, what=""):
    import torch

    g, r = bits(got), bits(ref)
    assert g.shape == r.shape, f"{what}: shape {tuple(g.shape)} vs {tuple(r.shape)}"
    if not torch.equal(g, r):
        diff = (g != r).nonzero()
        raise AssertionError(f"{what}: {diff.shape[0]} elements differ; first at {diff[0].tolist()}")
