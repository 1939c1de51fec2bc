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
