"""The R package integration files (integration/r): CPU checks.

R and Rcpp are not installed in this image, so the Rcpp sources are not
compiled here.  What can be checked without them:
  * the configure fragment lists the library's translation units and the
    library build's device and host flags (the perplexity search's bit-level
    agreement depends on -fno-gpu-flush-denormals-to-zero);
  * the objects it names link into one shared object with no undefined
    symbol (-Wl,--no-undefined), with R's C++ compiler (g++) as the linker;
  * it selects the stub when HIP is off and refuses other offload targets;
  * every C-ABI function the R implementation calls is declared in the
    header, and the bridge, implementation and stub define the same entry
    points.
"""

import os
import re
import shlex
import shutil
import subprocess
from pathlib import Path

import pytest

from fastembedr_amd import build

ROOT = Path(__file__).resolve().parent.parent
RDIR = ROOT / "integration" / "r"
FRAGMENT = RDIR / "configure.hip"
ROCM = Path(os.environ.get("ROCM_PATH", "/opt/rocm"))


def _source(env_extra: dict) -> tuple[int, dict]:
    env = {k: v for k, v in os.environ.items() if not k.startswith("FASTEMBEDR_")}
    env.update(env_extra)
    script = (f". {shlex.quote(str(FRAGMENT))}; "
              'printf "%s\\n" "$hip_enabled" "$hip_objects" "$hip_device_flags" "$hip_host_flags" "$cppflags" "$libs"')
    proc = subprocess.run(["sh", "-c", script], env=env, capture_output=True, text=True)
    if proc.returncode != 0:
        return proc.returncode, {"stderr": proc.stderr}
    lines = proc.stdout.split("\n")
    keys = ["enabled", "objects", "device", "host", "cppflags", "libs"]
    return 0, dict(zip(keys, lines))


def _hipcc_env():
    hipcc = ROCM / "bin" / "hipcc"
    if not hipcc.exists():
        pytest.skip("hipcc not present")
    return {"HIPCC": str(hipcc), "FASTEMBEDR_USE_HIP": "1", "ROCM_PATH": str(ROCM)}


def test_fragment_units_and_flags_match_the_library_build():
    rc, out = _source(_hipcc_env())
    assert rc == 0, out
    assert out["enabled"] == "1"
    objs = out["objects"].split()
    assert objs[0] == "embedding_hip_impl.o"
    units = [o[:-2] for o in objs[1:]]
    assert sorted(units) == sorted(build.HOST_UNITS + build.DEVICE_UNITS)
    device = out["device"].split()
    want = [f for f in build.DEVICE_FLAGS]
    assert device == want, (device, want)
    assert out["host"].split() == build.HOST_FLAGS
    assert "-DFASTEMBEDR_HAS_HIP" in out["cppflags"].split()
    assert "-lamdhip64" in out["libs"].split()


def test_fragment_stub_and_target_checks():
    rc, out = _source({"FASTEMBEDR_USE_HIP": "0", "HIPCC": "/nonexistent/hipcc"})
    assert rc == 0 and out["enabled"] == "0" and out["objects"] == "embedding_hip_stub.o"
    rc, out = _source({"FASTEMBEDR_USE_HIP": "1", "HIPCC": "", "ROCM_PATH": "/nonexistent"})
    assert rc != 0 and "no hipcc" in out["stderr"]
    env = _hipcc_env()
    env["FASTEMBEDR_HIP_ARCH"] = "gfx942"
    rc, out = _source(env)
    assert rc != 0 and "gfx950" in out["stderr"]


def test_fragment_objects_link_without_undefined_symbols(tmp_path):
    rc, out = _source(_hipcc_env())
    assert rc == 0, out
    units = [o[:-2] for o in out["objects"].split()[1:]]
    objs = [build.BUILD_DIR / f"{u}.o" for u in units]
    if not all(o.exists() for o in objs):
        build.build()
    cxx = shutil.which("g++")
    if cxx is None:
        pytest.skip("g++ not present")
    so = tmp_path / "libfastembedr_hip_rpkg.so"
    cmd = [cxx, "-shared", "-o", str(so), *map(str, objs), "-Wl,--no-undefined", f"-L{ROCM / 'lib'}",
           f"-Wl,-rpath,{ROCM / 'lib'}", "-lamdhip64"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-4000:]
    syms = subprocess.run(["nm", "-D", "--defined-only", str(so)], capture_output=True, text=True).stdout
    header = (ROOT / "include" / "fastembedr_hip.h").read_text()
    declared = set(re.findall(r"FASTEMBEDR_HIP_API\s+[\w\s\*]+?\b(fastembedr_hip_\w+)\s*\(", header))
    exported = set(re.findall(r"\bT (fastembedr_hip_\w+)", syms))
    assert declared and declared <= exported, declared - exported


def test_impl_calls_only_declared_abi_and_files_agree():
    header = (ROOT / "include" / "fastembedr_hip.h").read_text()
    declared = set(re.findall(r"FASTEMBEDR_HIP_API\s+[\w\s\*]+?\b(fastembedr_hip_\w+)\s*\(", header))
    impl = (RDIR / "src" / "embedding_hip_impl.cpp").read_text()
    called = set(re.findall(r"\b(fastembedr_hip_\w+)\s*\(", impl))
    assert called and called <= declared, called - declared
    entry = re.compile(r"^(?:bool|List|NumericMatrix)\s+(\w+_impl)\s*\(", re.M)
    bridge = set(entry.findall((RDIR / "src" / "embedding_hip_bridge.cpp").read_text()))
    stub = set(entry.findall((RDIR / "src" / "embedding_hip_stub.cpp").read_text()))
    defined = set(entry.findall(impl))
    assert bridge == stub == defined, (bridge, stub, defined)
    exports = set(re.findall(r"\b(\w+_cpp)\s*\(", (RDIR / "src" / "embedding_hip_bridge.cpp").read_text()))
    r_code = (RDIR / "R" / "hip_backend.R").read_text()
    used = set(re.findall(r"\b(\w+_hip\w*_cpp)\b", r_code))
    assert used <= exports, used - exports


def test_impl_checks_perplexity_before_either_route():
    """check_opt_args refuses n - 1 < 3 * perplexity (the CPU driver's rule,
    src/tsne_neighbors.cpp:1652) for both the one-shot route and the
    cost-recording session route, which calls it before branching."""
    impl = (RDIR / "src" / "embedding_hip_impl.cpp").read_text()
    body = impl[impl.index("void check_opt_args("):]
    body = body[:body.index("\n}\n")]
    assert re.search(r"n - 1\)\s*<\s*3\.0 \* a\.perplexity", body)
    assert "perplexity is too large for the number of samples." in body
    for entry in re.finditer(r"\nList (\w+_impl)\(", impl):
        fn = impl[entry.end():]
        fn = fn[:fn.index("\n}\n")]
        if "record_costs" in fn:
            assert fn.index("check_opt_args(") < fn.index("if (record_costs)"), entry.group(1)


# ---------------------------------------------------------------------------
# The hooks in the package's existing files, shipped as unified diffs
# against the reference's sources (integration/r/patches/)
# ---------------------------------------------------------------------------
REFERENCE = Path("/root/reference")
PATCHES = sorted((RDIR / "patches").glob("*.patch"))
HOOKED = ["configure", "R/backend_info.R", "R/fast_knn_tsne.R", "R/native_knn.R", "R/tsne_affinity_dispatch.R",
          "R/transform_tsne.R", "R/evaluate_embedding.R", "R/knn_input.R"]

# Switch points on the path that stay CUDA-only on purpose, with the reason.
CUDA_ONLY = {
    # device PCA initialisation (RAFT tSVD): the HIP route computes the PCA
    # initialisation on the host (opentsne_knn converts init_data to Y_init)
    ("R/fast_knn_tsne.R", "opentsne", "optimizer_backend"),
    ("R/tsne_affinity_dispatch.R", "fast_knn_opentsne_materialized", "optimizer_backend@cuda_init_data"),
    # query KNN stays on the host for HIP: its transform takes host matrices
    ("R/native_knn.R", "precompute_query_knn", "backend"),
}


def _patched_tree(tmp_path):
    if not REFERENCE.is_dir():
        pytest.skip("the reference sources are not present on this machine")
    if shutil.which("git") is None:
        pytest.skip("git not present")
    for rel in HOOKED:
        dst = tmp_path / rel
        dst.parent.mkdir(parents=True, exist_ok=True)
        shutil.copyfile(REFERENCE / rel, dst)
    proc = subprocess.run(["git", "apply", *map(str, PATCHES)], cwd=tmp_path, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr
    return tmp_path


def _functions(text):
    """Top-level R functions: name -> body text (up to the closing brace at
    column 0)."""
    out = {}
    for m in re.finditer(r"^([A-Za-z_.][\w.]*) <- function\(", text, re.M):
        end = text.find("\n}\n", m.end())
        out[m.group(1)] = text[m.end():end if end >= 0 else len(text)]
    return out


def test_patches_apply_to_the_reference_sources():
    """Every patch names one of the hooked files and applies cleanly to the
    reference's own copy (git apply --check touches nothing)."""
    if not REFERENCE.is_dir():
        pytest.skip("the reference sources are not present on this machine")
    if shutil.which("git") is None:
        pytest.skip("git not present")
    assert len(PATCHES) == len(HOOKED)
    named = set()
    for p in PATCHES:
        named |= set(re.findall(r"^\+\+\+ b/(\S+)", p.read_text(), re.M))
    assert named == set(HOOKED)
    proc = subprocess.run(["git", "apply", "--check", *map(str, PATCHES)], cwd=REFERENCE, capture_output=True,
                          text=True)
    assert proc.returncode == 0, proc.stderr


def test_every_cuda_switch_point_on_the_path_has_a_hip_branch(tmp_path):
    """In the patched files, each `identical(v, "cuda")` condition of the
    functions on the opentsne / KNN / transform / metrics path is matched by a
    HIP branch on the same variable (`identical(v, "hip")` or
    `v %in% c("cuda", "hip")`), except the listed CUDA-only ones; every
    backend default vector offers "hip"."""
    root = _patched_tree(tmp_path)
    path_functions = {
        "R/fast_knn_tsne.R": ["opentsne_knn", "opentsne"],
        "R/tsne_affinity_dispatch.R": ["fast_knn_opentsne_materialized", "fast_knn_opentsne_core"],
        "R/native_knn.R": ["fastembedr_has_gpu_knn_shape", "fastembedr_embedding_nn_policy",
                           "fastembedr_query_nn_policy", "fastembedr_nn_policy_engine", "precompute_knn",
                           "precompute_query_knn", "fastembedr_nn_without_self", "fastembedr_native_query_knn"],
        "R/transform_tsne.R": ["transform_tsne", "resolve_tsne_transform_backend"],
    }
    missing = []
    for rel, names in path_functions.items():
        fns = _functions((root / rel).read_text())
        for name in names:
            assert name in fns, (rel, name)
            body = fns[name]
            for var in sorted(set(re.findall(r'identical\(([\w$]+), "cuda"\)', body))):
                hip = (f'identical({var}, "hip")' in body or f'{var} %in% c("cuda", "hip")' in body)
                if not hip and (rel, name, var) not in CUDA_ONLY:
                    missing.append((rel, name, var))
            for m in re.finditer(r'identical\(([\w$]+), "cuda"\) &&[^\n]*cuda_init_data', body):
                assert (rel, name, f"{m.group(1)}@cuda_init_data") in CUDA_ONLY or (rel, name, m.group(1)) in CUDA_ONLY
            for m in re.finditer(r'backend = c\(("[^)]*")\)', body):
                assert '"hip"' in m.group(1), (rel, name, m.group(0))
    assert not missing, missing
    # residency-keyed code: a KNN object resident on the HIP device is a GPU
    # KNN, is copied back by the HIP bridge, and reaches the HIP optimizer
    native = _functions((root / "R/native_knn.R").read_text())
    assert 'c("cuda", "hip")' in native["fastembedr_has_gpu_knn_shape"]
    assert "native_hip_knn_to_host_cpp" in native["fastembedr_gpu_knn_to_host"]
    assert "native_hip_knn_cpp" in native["fastembedr_nn_without_self"]
    assert "native_hip_query_knn_cpp" in native["fastembedr_native_query_knn"]
    info = (root / "R/backend_info.R").read_text()
    assert '"hip")' in _functions(info)["embedding_backend_choices"]
    assert "hip_backend_info_row()" in _functions(info)["backend_info"]
    assert "hip_structure_metrics(" in (root / "R/evaluate_embedding.R").read_text()
    cfg = (root / "configure").read_text()
    assert ". ./configure.hip" in cfg and "$hip_rule" in cfg and "embedding_hip_bridge.o $hip_objects" in cfg


def test_patched_hooks_call_only_defined_helpers_and_exports(tmp_path):
    """The helpers the patched files call exist in R/hip_backend.R, and the
    Rcpp entry points they call are exported by the bridge."""
    root = _patched_tree(tmp_path)
    added = "\n".join(line[1:] for p in PATCHES if "configure" not in p.name for line in p.read_text().splitlines()
                      if line.startswith("+") and not line.startswith("+++"))
    helpers = set(re.findall(r"\b(\w*hip\w*)\s*\(", added)) - {"identical"}
    r_defs = set(_functions((RDIR / "R" / "hip_backend.R").read_text()))
    bridge = set(re.findall(r"\b(\w+_cpp)\s*\(", (RDIR / "src" / "embedding_hip_bridge.cpp").read_text()))
    unknown = {h for h in helpers if h not in r_defs and h not in bridge}
    assert not unknown, unknown
    # the R-level backend switch accepts "hip" and still resolves a caller's
    # untouched three-entry default vector to its first entry
    body = _functions((root / "R/backend_info.R").read_text())["resolve_embedding_backend"]
    assert "backend[[1L]]" in body and "match.arg(backend, choices)" in body


def test_configure_fragment_sets_the_default_goal():
    """Without the CUDA rule, the first HIP object rule must not become make's
    default goal."""
    rc, out = _source(_hipcc_env())
    assert rc == 0, out
    env = {k: v for k, v in os.environ.items() if not k.startswith("FASTEMBEDR_")}
    env.update(_hipcc_env())
    proc = subprocess.run(["sh", "-c", f'. {shlex.quote(str(FRAGMENT))}; printf "%s" "$hip_rule"'], env=env,
                          capture_output=True, text=True)
    rule = proc.stdout
    assert rule.index(".DEFAULT_GOAL := all") < rule.index(".o:")
