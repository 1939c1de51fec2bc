"""Deterministic synthetic inputs for the benchmark configurations.

The reference's benchmark data are R-generated (set.seed + rnorm), which
cannot be reproduced without R; this generator (numpy PCG64) is therefore
part of the specification of each configuration.  All consumers (CPU
oracle, HIP backend) are fed the same bytes.

Configurations (BASELINE.json "configs"):
  0: 10,000 x 50, 10 components, means ~ N(0, 5^2 I), unit std, equal weights
  1: 70,000 x 50, 10 components, means ~ N(0, 4^2 I), std ~ U[0.5, 1.5],
     weights ~ Dirichlet(5)
  2: 1,000,000 x 50, 50 components, means ~ N(0, 6^2 I), unit std
  4: 4,000,000 x 50, 200 components, weights ~ Dirichlet(0.3), means ~ N(0, 6^2 I),
     unit std (the mean spread is not stated for this configuration)
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np


@dataclass(frozen=True)
class MixtureSpec:
    n: int
    dim: int = 50
    components: int = 10
    mean_sd: float = 5.0
    std_range: tuple[float, float] | None = None  # per-component std ~ U[lo, hi]; None = unit
    dirichlet: float | None = None                 # component weights; None = equal


CONFIGS = {
    0: MixtureSpec(n=10_000, components=10, mean_sd=5.0),
    1: MixtureSpec(n=70_000, components=10, mean_sd=4.0, std_range=(0.5, 1.5), dirichlet=5.0),
    2: MixtureSpec(n=1_000_000, components=50, mean_sd=6.0),
    4: MixtureSpec(n=4_000_000, components=200, mean_sd=6.0, dirichlet=0.3),
}

# Run schedule shared by every configuration: perplexity 30, k = 90, 250
# early-exaggeration iterations (exaggeration 12, momentum 0.5) then 500
# iterations (momentum 0.8), learning rate n / 12 in both phases.
SCHEDULE = dict(perplexity=30.0, k=90, early_exaggeration_iter=250, n_iter=500, early_exaggeration=12.0,
                exaggeration=1.0, initial_momentum=0.5, final_momentum=0.8, min_gain=0.01, max_step_norm=5.0,
                # FFT settings of the configs (FIt-SNE / openTSNE names)
                interpolation_points=3, min_intervals=50, ints_in_interval=1.0)


def gaussian_mixture(spec: MixtureSpec, seed: int = 1, n: int | None = None) -> tuple[np.ndarray, np.ndarray]:
    """Returns (x float32 (n, dim), labels int32)."""
    rng = np.random.Generator(np.random.PCG64(seed))
    n = spec.n if n is None else n
    means = rng.normal(0.0, spec.mean_sd, size=(spec.components, spec.dim))
    if spec.std_range is None:
        stds = np.ones(spec.components)
    else:
        stds = rng.uniform(spec.std_range[0], spec.std_range[1], size=spec.components)
    if spec.dirichlet is None:
        weights = np.full(spec.components, 1.0 / spec.components)
    else:
        weights = rng.dirichlet(np.full(spec.components, spec.dirichlet))
    labels = rng.choice(spec.components, size=n, p=weights).astype(np.int32)
    x = np.empty((n, spec.dim), np.float32)
    chunk = 1 << 18
    for s in range(0, n, chunk):
        lab = labels[s:s + chunk]
        noise = rng.standard_normal(size=(lab.size, spec.dim))
        x[s:s + chunk] = (means[lab] + noise * stds[lab, None]).astype(np.float32)
    return x, labels


def mixture_queries(spec: MixtureSpec, n_query: int, seed: int = 1, query_seed: int = 2) -> np.ndarray:
    """New points from the same mixture as gaussian_mixture(spec, seed): the
    component means, stds and weights are drawn from `seed` exactly as there,
    the queries' labels and noise from an independent stream `query_seed`.
    Config 3 places 100,000 such points against the config-1 embedding."""
    rng = np.random.Generator(np.random.PCG64(seed))
    means = rng.normal(0.0, spec.mean_sd, size=(spec.components, spec.dim))
    if spec.std_range is None:
        stds = np.ones(spec.components)
    else:
        stds = rng.uniform(spec.std_range[0], spec.std_range[1], size=spec.components)
    if spec.dirichlet is None:
        weights = np.full(spec.components, 1.0 / spec.components)
    else:
        weights = rng.dirichlet(np.full(spec.components, spec.dirichlet))
    qrng = np.random.Generator(np.random.PCG64(query_seed))
    labels = qrng.choice(spec.components, size=n_query, p=weights)
    noise = qrng.standard_normal(size=(n_query, spec.dim))
    return (means[labels] + noise * stds[labels, None]).astype(np.float32)


def pca_init(x: np.ndarray, n_components: int = 2, target_sd: float = 1e-4) -> np.ndarray:
    """PCA scores, centred, scaled so that the largest column sd (n - 1) is
    target_sd (R/tsne_control.R:364-389 semantics).  Returns float32 (n, 2)."""
    xd = x.astype(np.float64)
    mu = xd.mean(axis=0)
    cov = np.zeros((x.shape[1], x.shape[1]))
    for s in range(0, x.shape[0], 1 << 18):
        blk = xd[s:s + (1 << 18)] - mu
        cov += blk.T @ blk
    w, v = np.linalg.eigh(cov)
    order = np.argsort(w)[::-1][:n_components]
    comps = v[:, order]
    # deterministic sign: largest-magnitude loading positive
    signs = np.sign(comps[np.argmax(np.abs(comps), axis=0), np.arange(n_components)])
    comps = comps * signs
    scores = (xd - mu) @ comps
    scores -= scores.mean(axis=0)
    scale = scores.std(axis=0, ddof=1).max()
    if np.isfinite(scale) and scale > 0:
        scores *= target_sd / scale
    return scores.astype(np.float32)


def exact_knn_numpy(x: np.ndarray, k: int, chunk: int = 1024) -> tuple[np.ndarray, np.ndarray]:
    """Exact Euclidean KNN excluding self; (indices int32, distances float32), (n, k)."""
    xd = x.astype(np.float64)
    sq = (xd * xd).sum(axis=1)
    n = x.shape[0]
    idx = np.empty((n, k), np.int32)
    dist = np.empty((n, k), np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        d2 = sq[s:e, None] + sq[None, :] - 2.0 * (xd[s:e] @ xd.T)
        np.maximum(d2, 0.0, out=d2)
        d2[np.arange(e - s), np.arange(s, e)] = np.inf
        part = np.argpartition(d2, k, axis=1)[:, :k]
        pd = np.take_along_axis(d2, part, axis=1)
        order = np.lexsort((part, pd), axis=1)
        idx[s:e] = np.take_along_axis(part, order, axis=1)
        dist[s:e] = np.sqrt(np.take_along_axis(pd, order, axis=1)).astype(np.float32)
    return idx, dist


def exact_knn_torch(x: np.ndarray, k: int, device: str = "cuda", chunk: int = 4096):
    """Exact Euclidean KNN excluding self, computed with torch on the GPU
    (input preparation only; not part of the t-SNE path).  Returns numpy
    (indices int32, distances float32), each (n, k)."""
    import torch

    xt = torch.as_tensor(x, device=device, dtype=torch.float32)
    sq = (xt * xt).sum(dim=1)
    n = xt.shape[0]
    idx = np.empty((n, k), np.int32)
    dist = np.empty((n, k), np.float32)
    for s in range(0, n, chunk):
        e = min(n, s + chunk)
        d2 = sq[s:e, None] + sq[None, :] - 2.0 * (xt[s:e] @ xt.T)
        d2.clamp_(min=0.0)
        d2[torch.arange(e - s, device=device), torch.arange(s, e, device=device)] = float("inf")
        vals, inds = torch.topk(d2, k, dim=1, largest=False, sorted=True)
        idx[s:e] = inds.to(torch.int32).cpu().numpy()
        dist[s:e] = vals.sqrt().cpu().numpy()
        del d2, vals, inds
    return idx, dist


def exact_knn_partitioned_torch(x: np.ndarray, labels: np.ndarray, k: int, device: str = "cuda",
                                chunk: int = 4096):
    """Exact Euclidean KNN excluding self, computed on the GPU with torch
    (input preparation only), searching each part of a partition of the rows
    (here the mixture components) and certifying the result.

    Within a part the search is brute force in the part's centred
    coordinates.  A row's k neighbours found there are exact when, for every
    other part c, the triangle-inequality bound ||x - mu_c|| - r_c (mu_c the
    part's mean, r_c its largest distance to it) exceeds the row's k-th
    distance: no row of c can then be closer.  Rows that fail the
    certificate, and rows of parts with no more than k rows, are searched by
    brute force over all rows.  Returns numpy (indices int32, distances
    float32), each (n, k), and the number of rows searched by brute force."""
    import torch

    xt = torch.as_tensor(x, device=device, dtype=torch.float32)
    n = xt.shape[0]
    idx = np.empty((n, k), np.int32)
    dist = np.empty((n, k), np.float32)
    lab = np.asarray(labels)
    parts = np.unique(lab)
    order = np.argsort(lab, kind="stable")
    bounds = np.searchsorted(lab[order], parts)
    ends = np.append(bounds[1:], n)
    kth = torch.full((n,), float("inf"), device=device)
    centers = torch.empty((parts.size, xt.shape[1]), device=device)
    radii = torch.empty(parts.size, device=device)
    brute = torch.zeros(n, dtype=torch.bool, device=device)
    for c, (b, e) in enumerate(zip(bounds, ends)):
        rows = torch.as_tensor(order[b:e], device=device, dtype=torch.int64)
        xc = xt[rows]
        mu = xc.mean(dim=0)
        xc = xc - mu
        centers[c] = mu
        sqc = (xc * xc).sum(dim=1)
        radii[c] = sqc.max().sqrt()
        size = rows.numel()
        if size <= k:
            brute[rows] = True
            continue
        for s in range(0, size, chunk):
            t = min(size, s + chunk)
            d2 = sqc[s:t, None] + sqc[None, :] - 2.0 * (xc[s:t] @ xc.T)
            d2.clamp_(min=0.0)
            d2[torch.arange(t - s, device=device), torch.arange(s, t, device=device)] = float("inf")
            vals, inds = torch.topk(d2, k, dim=1, largest=False, sorted=True)
            sel = rows[s:t]
            idx[sel.cpu().numpy()] = rows[inds].to(torch.int32).cpu().numpy()
            dv = vals.sqrt()
            dist[sel.cpu().numpy()] = dv.cpu().numpy()
            kth[sel] = dv[:, -1]
            del d2, vals, inds
    # certificate: distance to every other part's centre minus its radius
    part_of = torch.as_tensor(np.searchsorted(parts, lab), device=device, dtype=torch.int64)
    csq = (centers * centers).sum(dim=1)
    for s in range(0, n, 1 << 16):
        t = min(n, s + (1 << 16))
        xs = xt[s:t]
        dc = ((xs * xs).sum(dim=1)[:, None] + csq[None, :] - 2.0 * (xs @ centers.T)).clamp_(min=0.0).sqrt()
        lb = dc - radii[None, :]
        lb[torch.arange(t - s, device=device), part_of[s:t]] = float("inf")
        # margin for the fp32 rounding of both distance computations
        bad = lb.min(dim=1).values <= kth[s:t] * (1.0 + 1e-4) + 1e-4
        brute[s:t] |= bad
    fails = torch.nonzero(brute).flatten()
    if fails.numel():
        sq = (xt * xt).sum(dim=1)
        for s in range(0, fails.numel(), chunk):
            sel = fails[s:s + chunk]
            d2 = sq[sel, None] + sq[None, :] - 2.0 * (xt[sel] @ xt.T)
            d2.clamp_(min=0.0)
            d2[torch.arange(sel.numel(), device=device), sel] = float("inf")
            vals, inds = torch.topk(d2, k, dim=1, largest=False, sorted=True)
            idx[sel.cpu().numpy()] = inds.to(torch.int32).cpu().numpy()
            dist[sel.cpu().numpy()] = vals.sqrt().cpu().numpy()
            del d2, vals, inds
    return idx, dist, int(fails.numel())


def exact_query_knn_torch(reference: np.ndarray, query: np.ndarray, k: int, device: str = "cuda",
                          chunk: int = 4096):
    """Exact Euclidean KNN of query rows among reference rows, with torch on
    the GPU (input preparation for the transform).  Returns numpy (indices
    int32 0-based, distances float64), each (n_query, k)."""
    import torch

    rt = torch.as_tensor(reference, device=device, dtype=torch.float32)
    qt = torch.as_tensor(query, device=device, dtype=torch.float32)
    rsq = (rt * rt).sum(dim=1)
    nq = qt.shape[0]
    idx = np.empty((nq, k), np.int32)
    dist = np.empty((nq, k), np.float64)
    for s in range(0, nq, chunk):
        e = min(nq, s + chunk)
        q = qt[s:e]
        d2 = (q * q).sum(dim=1)[:, None] + rsq[None, :] - 2.0 * (q @ rt.T)
        d2.clamp_(min=0.0)
        vals, inds = torch.topk(d2, k, dim=1, largest=False, sorted=True)
        idx[s:e] = inds.to(torch.int32).cpu().numpy()
        dist[s:e] = vals.sqrt().double().cpu().numpy()
        del d2, vals, inds
    return idx, dist


def to_r_layout(indices: np.ndarray, distances: np.ndarray, one_based: bool = True):
    """(n, k) arrays -> column-major int32 / float32 as R would hand them over."""
    idx = np.asfortranarray(indices.astype(np.int32) + (1 if one_based else 0))
    dist = np.asfortranarray(distances.astype(np.float32))
    return idx, dist
