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


def poisson_binomial_pvalue(ps, k: int) -> float:
    """Two-sided p-value of observing k successes among independent Bernoulli(p_i) trials:
    the total probability of outcomes no more likely than k (exact, by dynamic programming
    over the trials)."""
    dist = np.zeros(len(ps) + 1)
    dist[0] = 1.0
    for i, p in enumerate(ps):
        nxt = dist * (1.0 - p)
        nxt[1:i + 2] += dist[:i + 1] * p
        dist = nxt
    return float(dist[dist <= dist[k] * (1 + 1e-9)].sum())


def chi_square_pvalue(samples, probs, min_expected: float = 5.0) -> float:
    """Goodness of fit of integer samples to a distribution over [0, len(probs)): Pearson's
    chi-square over the categories expected >= min_expected times, the rest (and any
    probability mass missing from probs) pooled into one category."""
    from scipy.stats import chi2

    n = len(samples)
    p = np.asarray(probs, dtype=np.float64)
    allc = np.bincount(np.asarray(samples, dtype=np.int64), minlength=len(p)).astype(np.float64)
    counts, beyond = allc[: len(p)], allc[len(p):].sum()
    exp = n * p
    big = exp >= min_expected
    obs_b, exp_b = list(counts[big]), list(exp[big])
    rest_o, rest_e = counts[~big].sum() + beyond, n - exp[big].sum()
    if rest_e > 0 or rest_o > 0:
        obs_b.append(rest_o)
        exp_b.append(max(rest_e, 1e-12))
    obs_b, exp_b = np.asarray(obs_b), np.asarray(exp_b)
    stat = float(((obs_b - exp_b) ** 2 / exp_b).sum())
    return float(chi2.sf(stat, max(1, len(obs_b) - 1)))
