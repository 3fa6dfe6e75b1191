"""Seeded inputs of the benchmark configurations (test infrastructure: see oracle/__init__.py).

Generated in float64 with numpy's default_rng; the same arrays go to the GPU path, the oracle and the CPU
baseline. Shapes and distributions follow the five workloads the reference's results are quoted on.
"""

from __future__ import annotations

import numpy as np


def mixture(n, d, k, seed, shift=0.0):
    """examples/sinkhorn_benchmark.py:38-43: n points from k Gaussian blobs (centres ~ N(0, 9 I))."""
    rng = np.random.default_rng(seed)
    centers = rng.normal(scale=3.0, size=(k, d))
    lab = rng.integers(k, size=n)
    return centers[lab] + rng.normal(size=(n, d)) + shift


def clouds(n=137, m=91, d=5, seed=0):
    """tests/test_sinkhorn.py:47-51: the reference tests' small clouds."""
    rng = np.random.default_rng(seed)
    x = rng.normal(size=(n, d))
    y = rng.normal(size=(m, d)) * 0.8 + 0.5
    return x, y


def balanced_gaussian(n=2048, m=2048, d=64, seed=0):
    """2048 x 2048, d 64, x, y ~ N(0, 1) from one generator (seed 0): the 100-iteration correctness workload."""
    r = np.random.default_rng(seed)
    return r.standard_normal((n, d)), r.standard_normal((m, d))


def synthetic_10k(n=10_000, m=10_000, d=64):
    """10k x 10k, d 64: x ~ N(0, 1) (seed 0), y ~ N(0, 1) + 0.5 (seed 1): the ms/iteration workload."""
    x = np.random.default_rng(0).standard_normal((n, d))
    y = np.random.default_rng(1).standard_normal((m, d)) + 0.5
    return x, y


def single_cell_like(n=7355, m=8962, d=30):
    """Anisotropic Gaussians with per-axis std 1/sqrt(k+1) (PCA-like), target mean offset 0.3 sigma, and
    lognormal(0, 0.5) source growth weights normalised to 1: the unbalanced single-cell-shaped workload."""
    sig = 1.0 / np.sqrt(np.arange(d) + 1.0)
    x = np.random.default_rng(0).standard_normal((n, d)) * sig
    y = np.random.default_rng(1).standard_normal((m, d)) * sig + 0.3 * sig
    w = np.random.default_rng(2).lognormal(0.0, 0.5, n)
    return x, y, w / w.sum()


def gaussian_mixture_8(n=65_536, m=65_536, d=128):
    """8-component mixture, component std 0.5, means ~ N(0, 4 I): the eps-scaling stress workload."""
    r = np.random.default_rng(0)
    mu = 2.0 * r.standard_normal((8, d))
    x = mu[r.integers(8, size=n)] + 0.5 * r.standard_normal((n, d))
    r1 = np.random.default_rng(1)
    y = mu[r1.integers(8, size=m)] + 0.5 * r1.standard_normal((m, d))
    return x, y
