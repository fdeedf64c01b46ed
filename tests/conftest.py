"""Shared fixtures for the CPU (oracle, host logic, ABI) and GPU (parity) suites."""

from __future__ import annotations

import math
import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
PKG = os.path.join(ROOT, "pulsar-300m_amd")
for p in (ROOT, PKG):
    if p not in sys.path:
        sys.path.insert(0, p)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def gpu_available() -> bool:
    return torch.cuda.is_available()


@pytest.fixture(scope="session")
def full_state():
    """Synthetic fp32 weights of the full-size model (seed 0), generated once per session."""
    from pulsar_engine import weights as W
    from pulsar_engine.config import PulsarConfig

    cfg = PulsarConfig()
    return cfg, W.synthetic_state(cfg, seed=0)


@pytest.fixture(scope="session")
def models(full_state):
    """The full-size synthetic model on the GPU in fp32 and bf16, shared by the GPU suites."""
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    from pulsar_engine.model import DeviceModel

    cfg, st = full_state
    return {
        torch.float32: DeviceModel(cfg, st, torch.float32),
        torch.bfloat16: DeviceModel(cfg, st, torch.bfloat16),
    }


@pytest.fixture(scope="session")
def tiny_state():
    from pulsar_engine import weights as W
    from pulsar_engine.config import tiny_config

    cfg = tiny_config()
    return cfg, W.synthetic_state(cfg, seed=0)


def golden(name: str):
    return np.load(os.path.join(GOLDEN, name))


def assert_close(actual, expected, *, atol=2e-2, rtol=2e-2, msg=""):
    """Passes when either the absolute or the relative bound holds everywhere."""
    a = torch.as_tensor(actual).detach().float().cpu()
    e = torch.as_tensor(expected).detach().float().cpu()
    assert a.shape == e.shape, f"{msg}: shape {tuple(a.shape)} vs {tuple(e.shape)}"
    if a.numel() == 0:
        return
    diff = (a - e).abs()
    max_abs = diff.max().item()
    max_rel = (diff / e.abs().clamp_min(1e-6)).max().item()
    assert math.isfinite(max_abs), f"{msg}: non-finite values"
    assert max_abs <= atol or max_rel <= rtol, (
        f"{msg}: max_abs={max_abs:.3e} (atol {atol:.1e}) max_rel={max_rel:.3e} (rtol {rtol:.1e})")


def max_abs_rel(actual, expected) -> float:
    """max|a-e| / max|e| (the logits criterion)."""
    a = torch.as_tensor(actual).float()
    e = torch.as_tensor(expected).float()
    return ((a - e).abs().max() / e.abs().max().clamp_min(1e-12)).item()
