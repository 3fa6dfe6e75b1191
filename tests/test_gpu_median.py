"""The exact cost median on the GPU (sk_cost_median_f64), the normalisation of normalize="median"
(src/trnopt/sinkhorn.py:229-233), against np.median of the dense float64 cost matrix.

With integer coordinates every cost is an exact float64 integer whatever the summation order, so the GPU's
order statistics must equal numpy's bit for bit; with real-valued coordinates the two compute the dot
products in different orders and agree to rounding (1e-12 relative)."""

import numpy as np
import pytest

from oracle import data

pytestmark = pytest.mark.gpu


def dense_median(xc, yc):
    """What the reference's normalization(how="median") takes the median of (src/trnopt/sinkhorn.py:229-233)."""
    C = ((xc * xc).sum(1)[:, None] + (yc * yc).sum(1)[None, :] - 2.0 * (xc @ yc.T)).ravel()
    return float(np.median(np.maximum(C, 0.0)))


@pytest.mark.parametrize("n,m,d,lo,hi", [(1, 1, 1, -5, 5), (3, 5, 2, -9, 9), (4, 6, 3, -9, 9), (37, 129, 7, -3, 3),
                                         (300, 257, 30, -40, 40), (513, 100, 100, -2, 2), (64, 65, 128, -1, 1),
                                         (1000, 999, 5, 0, 1)])
def test_integer_clouds_match_numpy_exactly(hip, n, m, d, lo, hi):
    rng = np.random.default_rng(n * 1000 + m)
    x = rng.integers(lo, hi + 1, size=(n, d)).astype(np.float64)
    y = rng.integers(lo, hi + 1, size=(m, d)).astype(np.float64)
    print("median", n, m, d, flush=True)
    got = hip.cost_median(x, y, "cuda")
    assert got == dense_median(x, y)


def test_identical_clouds_have_zero_costs(hip):
    x = np.random.default_rng(0).integers(-2, 3, size=(50, 4)).astype(np.float64)
    got = hip.cost_median(x, x.copy(), "cuda")
    assert got == dense_median(x, x)


@pytest.mark.parametrize("n", [2000, 2100])
def test_two_tied_costs_across_the_middle_ranks(hip, n):
    """n x n pairs of two costs, 0 and 1, split so that the two middle ranks fall on different ones (median 0.5).
    Every key matches a rank's prefix in the third pass, which collects them for the last three: 4.0M keys fit
    the 2^22 it keeps; 4.41M do not, and the last passes recompute every cost instead."""
    x = np.tile([1.0, 2.0, 3.0], (n, 1))
    y = x.copy()
    y[n // 2:, 2] = 4.0
    print("tied median", n, flush=True)
    got = hip.cost_median(x, y, "cuda")
    assert got == dense_median(x, y) == 0.5


def test_single_cell_shaped_median_matches_the_reference_host_routine(hip):
    """The unbalanced single-cell workload's cost (7,355 x 8,962, d 30): the GPU median against the host
    normalisation the reference runs (one 527 MB float64 matrix)."""
    from trnopt.sinkhorn import normalization
    x, y, _ = data.single_cell_like()
    print("single-cell median", flush=True)
    c_gpu, s_gpu = normalization(x, y, how="median", device="cuda")
    c_cpu, s_cpu = normalization(x, y, how="median")
    np.testing.assert_array_equal(c_gpu, c_cpu)
    assert abs(s_gpu - s_cpu) <= 1e-12 * s_cpu, (s_gpu, s_cpu)


@pytest.mark.parametrize("d", [1, 33, 64, 128])
def test_real_valued_clouds_agree_to_rounding(hip, d):
    rng = np.random.default_rng(d)
    x = rng.standard_normal((700, d)) * 3.0
    y = rng.standard_normal((455, d)) + 0.25
    got = hip.cost_median(x, y, "cuda")
    want = dense_median(x, y)
    assert abs(got - want) <= 1e-12 * want


def test_rejected_shapes(hip):
    x = np.zeros((4, 129))
    with pytest.raises(ValueError):
        hip.cost_median(x, x, "cuda")


def test_solver_uses_the_gpu_median(hip):
    from trnopt import Backend
    from trnopt.sinkhorn import SinkhornOptions, normalization, sinkhorn
    x, y = data.clouds(n=400, m=300, d=6, seed=2)
    res = sinkhorn(x, y, opts=SinkhornOptions(kernel="hip", backend=Backend.preset("rocm"), normalize="median",
                                             eps=0.1, max_iters=50, fixed_iters=True))
    assert abs(res.cost_scale - normalization(x, y, how="median")[1]) <= 1e-12 * res.cost_scale


def test_median_normalizations_equal_the_one_pair_calls(hip):
    """median_normalizations (a pipeline's pairs, every exact median enqueued at once, one read-back) gives each
    pair's normalization(how="median", device) bit for bit, including a pair above the exact median's 1e8 cost
    pairs, which takes the sampled median on the host as the one-pair call does."""
    import torch
    from trnopt.sinkhorn import median_normalizations, normalization
    dev = torch.device("cuda", 0)
    pairs = [data.clouds(n=n, m=m, d=d, seed=s) for n, m, d, s in ((300, 257, 30, 1), (40, 900, 7, 2), (1, 1, 3, 3),
                                                                   (1200, 1100, 64, 4))]
    rng = np.random.default_rng(5)
    pairs.append((rng.normal(size=(10_001, 2)), rng.normal(size=(10_000, 2))))    # 1.00001e8 pairs
    got = median_normalizations(pairs, dev)
    for (x, y), (c, s) in zip(pairs, got):
        c1, s1 = normalization(x, y, how="median", device=dev)
        np.testing.assert_array_equal(c, c1)
        assert s == s1, (s, s1)
