"""Exact structure metrics on the GPU (metrics_hip.hip through
fastembedr_hip_structure_metrics) against the CPU oracle restating
exact_structure_metrics_cpp (src/embedding_utils.cpp:1582-1752).

The squared distances are formed in the reference's operation order, so the
rankings and hence the metrics must be identical (assert_array_equal), ties
included."""

import sys

import numpy as np
import pytest

from fastembedr_amd import _lib
from oracle import metrics_oracle as mo

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)
    sys.stdout.flush()


def _gpu(high, low, ks):
    from fastembedr_amd.metrics import COLUMNS, exact_structure_metrics

    r = exact_structure_metrics(high, low, ks)
    return np.stack([r[c] for c in COLUMNS], axis=1)


@pytest.mark.parametrize("n,p,ks", [(2000, 50, [15, 30, 50]), (300, 7, [5]), (5000, 10, [15])])
def test_matches_oracle(hip, n, p, ks):
    _say(f"case: structure metrics n={n} p={p} k={ks}")
    rng = np.random.default_rng(n)
    centres = rng.normal(scale=4.0, size=(6, p))
    high = centres[rng.integers(0, 6, size=n)] + rng.normal(size=(n, p))
    low = high[:, :2] + rng.normal(scale=0.5, size=(n, 2))
    np.testing.assert_array_equal(_gpu(high, low, ks), mo.exact_structure_metrics(high, low, ks))


def test_ties_and_identity(hip):
    _say("case: structure metrics with ties and an identical layout")
    rng = np.random.default_rng(7)
    high = rng.integers(0, 3, size=(400, 4)).astype(float)
    low = rng.integers(0, 5, size=(400, 2)).astype(float)
    np.testing.assert_array_equal(_gpu(high, low, [10, 20]), mo.exact_structure_metrics(high, low, [10, 20]))
    x = rng.normal(size=(500, 2))
    m = _gpu(x, x, [15])
    np.testing.assert_array_equal(m[0], [1.0, 1.0, 1.0, 0.0])


def test_errors(hip):
    _say("case: structure metrics errors")
    x = np.zeros((10, 2))
    with pytest.raises(_lib.HipBackendError, match="each k must satisfy"):
        _gpu(x, x, [7])
    with pytest.raises(_lib.HipBackendError, match="at most 5000"):
        _gpu(np.zeros((5001, 2)), np.zeros((5001, 2)), [15])
    with pytest.raises(_lib.HipBackendError, match="three observations"):
        _gpu(np.zeros((2, 2)), np.zeros((2, 2)), [1])
