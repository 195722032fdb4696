"""Shared fixtures: the product package (loaded from its directory), the CPU
oracle, and GPU helpers.  Tests marked `gpu` need a ROCm device; everything
else runs on the CPU."""
from __future__ import annotations

import importlib.util
import pathlib
import sys

import numpy as np
import pytest

ROOT = pathlib.Path(__file__).resolve().parent.parent
PKG_DIR = ROOT / "inferencer-jetson_amd"
PKG_NAME = "inferencer_jetson_amd"


def load_package():
    if PKG_NAME in sys.modules:
        return sys.modules[PKG_NAME]
    spec = importlib.util.spec_from_file_location(PKG_NAME, PKG_DIR / "__init__.py",
                                                  submodule_search_locations=[str(PKG_DIR)])
    mod = importlib.util.module_from_spec(spec)
    sys.modules[PKG_NAME] = mod
    spec.loader.exec_module(mod)
    return mod


def load_oracle():
    if str(ROOT / "oracle") not in sys.path:
        sys.path.insert(0, str(ROOT / "oracle"))
    import oracle  # noqa: E402
    return oracle


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X / gfx950)")


@pytest.fixture(scope="session")
def qk():
    return load_package()


@pytest.fixture(scope="session")
def synth(qk):
    import inferencer_jetson_amd.synth as s
    return s


@pytest.fixture(scope="session")
def workloads(qk):
    import inferencer_jetson_amd.workloads as w
    return w


@pytest.fixture(scope="session")
def oracle():
    return load_oracle()


@pytest.fixture(scope="session")
def torch_gpu():
    import torch
    if not torch.cuda.is_available():
        pytest.fail("GPU test run without a visible GPU")
    return torch


def rel_l2(a, b) -> float:
    a = np.asarray(a, dtype=np.float64)
    b = np.asarray(b, dtype=np.float64)
    den = np.linalg.norm(b)
    return float(np.linalg.norm(a - b) / (den if den > 0 else 1.0))


def to_dev(torch, arr):
    """numpy -> device tensor (same dtype, contiguous)."""
    return torch.from_numpy(np.ascontiguousarray(arr)).to("cuda")
