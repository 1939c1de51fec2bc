"""The bench's input preparation: the partitioned, certified exact KNN must
equal brute force (numpy, fp64) on the same rows, whether the certificate
holds for every row (separated mixture components) or fails for many
(a random partition, searched again by brute force)."""

import numpy as np

from fastembedr_amd import synthetic


def _check(x, labels, k):
    idx, dist, brute = synthetic.exact_knn_partitioned_torch(x, labels, k, device="cpu", chunk=512)
    ref_idx, ref_dist = synthetic.exact_knn_numpy(x, k)
    np.testing.assert_allclose(dist, ref_dist, rtol=1e-4, atol=1e-4)
    # identical neighbour sets except where distances tie at rounding level
    same = np.mean(np.sort(idx, axis=1) == np.sort(ref_idx, axis=1))
    assert same > 0.999, same
    assert not np.any(idx == np.arange(x.shape[0])[:, None])
    return brute


def test_partitioned_knn_separated_components():
    spec = synthetic.MixtureSpec(n=3000, dim=20, components=8, mean_sd=6.0, dirichlet=0.3)
    x, labels = synthetic.gaussian_mixture(spec, seed=5)
    brute = _check(x, labels, 30)
    # small parts (<= k rows) and uncertified rows are the only brute-force rows
    sizes = np.bincount(labels, minlength=8)
    assert brute <= int(sizes[sizes <= 30].sum()) + 30


def test_partitioned_knn_random_partition_falls_back():
    spec = synthetic.MixtureSpec(n=2000, dim=10, components=4, mean_sd=3.0)
    x, _ = synthetic.gaussian_mixture(spec, seed=7)
    labels = np.random.default_rng(0).integers(0, 5, size=2000).astype(np.int32)
    brute = _check(x, labels, 25)
    assert brute > 1000


def test_mixture_queries_share_the_mixture():
    """Config 3's queries come from config 1's mixture: each query lies within
    a few component stds of one of the components' means (estimated from the
    labelled rows), while a mixture drawn from another seed is far off."""
    spec = synthetic.CONFIGS[1]
    x, labels = synthetic.gaussian_mixture(spec, seed=1, n=20000)
    means = np.stack([x[labels == c].mean(axis=0) for c in range(spec.components)])

    def nearest_d2(q):
        d2 = (q ** 2).sum(1)[:, None] - 2 * q @ means.T + (means ** 2).sum(1)[None, :]
        return d2.min(axis=1)

    q = synthetic.mixture_queries(spec, 3000)
    other = synthetic.mixture_queries(spec, 3000, seed=2)
    # within-component squared distance ~ dim * std^2 <= 50 * 1.5^2
    assert np.median(nearest_d2(q.astype(np.float64))) < 130.0
    assert np.median(nearest_d2(other.astype(np.float64))) > 500.0
    np.testing.assert_array_equal(q, synthetic.mixture_queries(spec, 3000))
