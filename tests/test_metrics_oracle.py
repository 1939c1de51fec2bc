"""Pins of the structure-metrics oracle (oracle/metrics_oracle.py), which
restates exact_structure_metrics_cpp (src/embedding_utils.cpp:1582-1752)."""

import numpy as np
import pytest

from oracle import metrics_oracle as mo


@pytest.mark.parametrize("n,k,seed", [(9, 2, 0), (14, 4, 1), (20, 6, 2)])
def test_matches_brute_force(n, k, seed):
    rng = np.random.default_rng(seed)
    high = rng.integers(0, 4, size=(n, 5)).astype(float)  # ties in the high space
    low = rng.normal(size=(n, 2))
    np.testing.assert_array_equal(mo.exact_structure_metrics(high, low, [k])[0], mo.brute_force_metrics(high, low, k))


def test_identity_and_invariance():
    rng = np.random.default_rng(3)
    x = rng.normal(size=(60, 2))
    m = mo.exact_structure_metrics(x, x, [5, 15])
    np.testing.assert_array_equal(m[:, :3], 1.0)
    np.testing.assert_array_equal(m[:, 3], 0.0)
    high = rng.normal(size=(60, 8))
    base = mo.exact_structure_metrics(high, x, [5, 10])
    c, s = np.cos(0.7), np.sin(0.7)
    rot = x @ np.array([[c, -s], [s, c]]) + 3.0
    np.testing.assert_allclose(mo.exact_structure_metrics(high, rot, [5, 10]), base, atol=1e-12)


def test_line_reversal_closed_form():
    # points on a line and their mirror image: identical neighbourhoods
    t = np.arange(30, dtype=float)[:, None] * 1.37
    m = mo.exact_structure_metrics(t, -t, [3])
    assert m[0, 2] == 1.0 and m[0, 0] == 1.0 and m[0, 1] == 1.0


def test_rejects_bad_k():
    x = np.zeros((10, 2))
    with pytest.raises(ValueError):
        mo.exact_structure_metrics(x, x, [7])
