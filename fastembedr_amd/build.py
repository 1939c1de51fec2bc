"""Builds the gfx950 HIP library in-tree (fastembedr_amd/lib/libfastembedr_hip.so).

The library is plain HIP C++ behind the C ABI of include/fastembedr_hip.h;
nothing in it depends on torch.  Run ``python -m fastembedr_amd.build``.
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG = Path(__file__).resolve().parent
ROOT = PKG.parent
CSRC = PKG / "csrc"
LIB_DIR = PKG / "lib"
LIB = LIB_DIR / "libfastembedr_hip.so"
BUILD_DIR = ROOT / "_build" / "hip"

ARCH = os.environ.get("FASTEMBEDR_HIP_ARCH", "gfx950")

# Device-code flags.  Packed fp32 instructions are switched off (they have
# given silent wrong results on these boxes); denormals are kept so that the
# perplexity search matches a CPU build bit for bit wherever exp/log agree.
DEVICE_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-fvisibility=hidden",
    "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
]
HOST_FLAGS = ["-O2", "-std=c++17", "-fPIC", "-fvisibility=hidden", "-Wall", "-D__HIP_PLATFORM_AMD__"]

# Translation units: device code (hipcc with DEVICE_FLAGS) and the host
# orchestration (hipcc with HOST_FLAGS).  The R package's configure fragment
# (integration/r/configure.hip) lists the same units and flags.
DEVICE_UNITS = ("embedding_hip_kernels", "attraction_tiles_hip", "transform_hip", "interp_grid_hip", "knn_hip",
                "metrics_hip")
HOST_UNITS = ("embedding_hip_session",)


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def _run(cmd: list[str]) -> None:
    print("+", " ".join(cmd), flush=True)
    subprocess.run(cmd, check=True)


def build(verbose: bool = True) -> Path:
    hipcc = _hipcc()
    BUILD_DIR.mkdir(parents=True, exist_ok=True)
    LIB_DIR.mkdir(parents=True, exist_ok=True)
    inc = ["-I", str(ROOT / "include"), "-I", str(CSRC)]
    objs = []
    jobs = [([hipcc, *DEVICE_FLAGS, *inc, "-c", str(CSRC / f"{name}.hip"), "-o", str(BUILD_DIR / f"{name}.o")],
             BUILD_DIR / f"{name}.o") for name in DEVICE_UNITS]
    jobs += [([hipcc, *HOST_FLAGS, *inc, "-c", str(CSRC / f"{name}.cpp"), "-o", str(BUILD_DIR / f"{name}.o")],
              BUILD_DIR / f"{name}.o") for name in HOST_UNITS]
    # the units compile independently: run them side by side
    workers = max(1, min(len(jobs), int(os.environ.get("MAX_JOBS", "0")) or (os.cpu_count() or 1)))
    pending = list(jobs)
    running = []
    while pending or running:
        while pending and len(running) < workers:
            cmd, _ = pending.pop(0)
            print("+", " ".join(cmd), flush=True)
            running.append((cmd, subprocess.Popen(cmd)))
        cmd, proc = running.pop(0)
        if proc.wait() != 0:
            for _, other in running:
                other.wait()
            raise subprocess.CalledProcessError(proc.returncode, cmd)
    objs = [str(obj) for _, obj in jobs]
    tmp = LIB.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objs, "-o", str(tmp)])
    os.replace(tmp, LIB)
    return LIB


def build_oracle() -> Path:
    _run(["make", "-s", "-C", str(ROOT / "oracle")])
    return ROOT / "oracle" / "_build" / "libtsne_oracle.so"


if __name__ == "__main__":
    build()
    if "--oracle" in sys.argv:
        build_oracle()
