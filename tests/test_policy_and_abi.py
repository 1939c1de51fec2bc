"""Host logic and the C-ABI surface (no GPU compute calls)."""

import ctypes
import json
import re
from pathlib import Path

import numpy as np
import pytest

import fastembedr_amd as fe
from fastembedr_amd import _lib, opentsne, synthetic

ROOT = Path(__file__).resolve().parent.parent


GOLDEN = json.loads((ROOT / "tests" / "golden" / "reference_test_constants.json").read_text())


@pytest.mark.parametrize("case", GOLDEN["auto_parameters"], ids=lambda c: f"n{c['n']}_k{c['k']}")
def test_auto_parameters_match_reference_constants(case):
    # constants asserted by the reference's tests/testthat/test-tsne.R:31-56
    p = fe.tsne_auto_parameters(case["n"], case["k"], case["perplexity_in"])
    for key, want in case["expect"].items():
        if key == "learning_rate_is_n_over_early_exaggeration":
            assert (p["learning_rate"] == case["n"] / p["early_exaggeration"]) is want
        else:
            assert p[key] == want, key


def test_auto_parameters_schedule():
    big = fe.tsne_auto_parameters(70000, 90, None)
    assert big["early_exaggeration"] == 12.0
    assert big["early_exaggeration_iter"] == 250 and big["n_iter"] == 500


def test_result_labels_follow_reference_naming():
    lab = GOLDEN["labels"]
    # The HIP labels take the CUDA backend's naming with the backend swapped.
    assert opentsne.OPTIMIZER_LABEL == lab["cuda_optimizer"].replace("_cuda", "_hip")
    assert opentsne.REPULSION_LABEL == "fft_grid_hip"
    assert opentsne.OPTIMIZER_LABEL.startswith("opentsne_fitsne_fft_grid")


def test_neighbor_policy():
    assert fe.opentsne_neighbor_policy(100, None, 20) == dict(perplexity=None, n_neighbors=15)
    assert fe.opentsne_neighbor_policy(1000, 30.0, 90)["n_neighbors"] == 30
    with pytest.raises(ValueError, match="no larger than"):
        fe.opentsne_neighbor_policy(50, 20.0, 30)
    with pytest.raises(ValueError, match="fewer non-self columns"):
        fe.opentsne_neighbor_policy(1000, 30.0, 20)


def test_strip_self_neighbors():
    n, k = 50, 6
    rng = np.random.default_rng(0)
    others = [rng.permutation(np.delete(np.arange(n), i))[: k - 1] for i in range(n)]
    idx = np.concatenate([np.arange(n)[:, None], np.stack(others)], axis=1) + 1
    dist = np.sort(rng.random((n, k)).astype(np.float32), axis=1)
    dist[:, 0] = 0.0
    i2, d2, has = opentsne.strip_self_neighbors(idx, dist)
    assert has and i2.shape == (n, k - 1)
    np.testing.assert_array_equal(i2, idx[:, 1:])
    # self not in the first column: removed where it is
    idx3 = idx.copy()
    idx3[:, [0, 2]] = idx3[:, [2, 0]]
    dist3 = dist.copy()
    dist3[:, [0, 2]] = dist3[:, [2, 0]]
    i3, d3, has3 = opentsne.strip_self_neighbors(idx3, dist3)
    assert has3 and not np.any(i3 == (np.arange(n) + 1)[:, None])
    # no self anywhere: unchanged
    i4, _, has4 = opentsne.strip_self_neighbors(idx[:, 1:], dist[:, 1:])
    assert not has4 and i4.shape == (n, k - 1)


def test_index_offset():
    assert opentsne.knn_index_offset(np.array([[1, 2], [2, 1]])) == 1
    assert opentsne.knn_index_offset(np.array([[0, 1], [1, 0]])) == 0


def test_method_aliases():
    assert opentsne.normalize_negative_gradient_method("auto") == "fft"
    assert opentsne.normalize_negative_gradient_method("FIt-SNE") == "fft"
    with pytest.raises(ValueError, match="removed"):
        opentsne.normalize_negative_gradient_method("bh")
    with pytest.raises(ValueError, match="changes the optimization mathematics"):
        opentsne.normalize_negative_gradient_method("sampled")
    with pytest.raises(ValueError, match="supports .*fft.* only"):
        opentsne.normalize_negative_gradient_method("exact")


def test_other_backends_refused_without_fallback():
    with pytest.raises(ValueError, match="No CPU fallback"):
        fe.opentsne_knn(np.zeros((5, 2), int), np.zeros((5, 2)), backend="cpu")


def _declared_symbols():
    text = (ROOT / "include" / "fastembedr_hip.h").read_text()
    return sorted(set(re.findall(r"FASTEMBEDR_HIP_API\s+[\w\s\*]+?\b(fastembedr_hip_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    declared = _declared_symbols()
    assert len(declared) >= 20
    lib = _lib.load()  # loads without touching a device
    for name in declared:
        assert hasattr(lib, name), name
    assert set(declared) == set(_lib.SIGNATURES), set(declared) ^ set(_lib.SIGNATURES)


def test_missing_library_fails_loudly(tmp_path):
    with pytest.raises(_lib.HipBackendUnavailable, match="No CPU fallback"):
        _lib.load(tmp_path / "missing.so")


def test_synthetic_generator_is_deterministic():
    spec = synthetic.MixtureSpec(n=1000, components=5, mean_sd=3.0, std_range=(0.5, 1.5), dirichlet=2.0)
    a, la = synthetic.gaussian_mixture(spec, seed=7)
    b, lb = synthetic.gaussian_mixture(spec, seed=7)
    np.testing.assert_array_equal(a, b)
    np.testing.assert_array_equal(la, lb)
    assert a.dtype == np.float32 and a.shape == (1000, 50)
    y = synthetic.pca_init(a)
    assert y.shape == (1000, 2)
    assert abs(y.std(axis=0, ddof=1).max() - 1e-4) < 1e-9
    np.testing.assert_allclose(y.mean(axis=0), 0, atol=1e-10)


def test_exact_knn_numpy_against_sklearn():
    from sklearn.neighbors import NearestNeighbors

    spec = synthetic.MixtureSpec(n=800, dim=10, components=3)
    x, _ = synthetic.gaussian_mixture(spec, seed=2)
    idx, dist = synthetic.exact_knn_numpy(x, 12)
    nn = NearestNeighbors(n_neighbors=13).fit(x.astype(np.float64))
    d_ref, i_ref = nn.kneighbors(x.astype(np.float64))
    np.testing.assert_allclose(dist, d_ref[:, 1:], rtol=1e-5, atol=1e-5)
    assert (idx == i_ref[:, 1:]).mean() > 0.999


def test_rocprof_digest_window(tmp_path):
    """The digests' --last N keeps the dispatches enqueued after the update
    that precedes the last N iterations: an FFT kernel instantiated for a
    length used only earlier in the run drops out, and each kernel keeps at
    most N dispatches."""
    from fastembedr_amd import rocprof_summary as rs

    rows = []
    did = 0

    def add(name, value):
        nonlocal did
        did += 1
        rows.append({"Dispatch_Id": str(did), "Kernel_Name": name, "Counter_Name": "FETCH_SIZE",
                     "Counter_Value": str(value)})

    add("__amd_rocclr_copyBuffer", 262166.6)
    for it in range(6):  # lengths 512 in iterations 0-2, 768 in 3-5
        fft = 512 if it < 3 else 768
        add(f"void fehip::(anonymous namespace)::k_lg_conv_cols<{fft}>(...)", fft)
        add("void fehip::(anonymous namespace)::k_attract_tiles_seg<512, 2, 3, false>(...)", 1000 + it)
        add("void fehip::k_update<0, true>(...)", 50)
    d = tmp_path / "pmc" / "sub"
    d.mkdir(parents=True)
    with open(d / "fetch_counter_collection.csv", "w") as f:
        f.write("Dispatch_Id,Kernel_Name,Counter_Name,Counter_Value\n")
        for r in rows:
            f.write(f'{r["Dispatch_Id"]},"{r["Kernel_Name"]}",{r["Counter_Name"]},{r["Counter_Value"]}\n')
    per, calib = rs._counter(str(tmp_path / "pmc"), "FETCH_SIZE", last=2)
    assert calib == pytest.approx(262166.6)
    assert "k_lg_conv_cols<512>" not in per
    assert per["k_lg_conv_cols<768>"] == [768.0, 768.0]
    assert per["k_attract_tiles_seg<512, 2, 3, false>"] == [1004.0, 1005.0]
    per_all, _ = rs._counter(str(tmp_path / "pmc"), "FETCH_SIZE", last=0)
    assert per_all["k_lg_conv_cols<512>"] == [512.0] * 3
