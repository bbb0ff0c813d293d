"""Build ``libflashdec_hip.so`` (the C-ABI library) in-tree with hipcc for gfx950,
and ``libflashdec_probe.so`` (bench.py's floor probes, ``csrc/floor_probe.hip``).

Each ``csrc/*.hip`` file is compiled separately, then linked into
``flashdec_amd/libflashdec_hip.so``.  The RoPE/append file is compiled with
FMA contraction disabled: its rotation must round every product and sum
separately to stay bit-exact against the oracle.  Both kernel files are
compiled with kernel-argument preloading: a kernel's leading scalar arguments
(up to 14 SGPRs) are written into SGPRs by the command processor at wave
launch, so short kernels issue their first loads without a kernel-argument
round trip.
"""

from __future__ import annotations

import os
import shutil
import subprocess
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB_PATH = PACKAGE_DIR / "libflashdec_hip.so"
# measurement probes for bench.py's floor workload (not the decode library)
PROBE_SOURCE = "floor_probe.hip"
PROBE_LIB_PATH = PACKAGE_DIR / "libflashdec_probe.so"
ARCH = "gfx950"

SOURCES = {
    "capi.hip": [],
    "paged_decode.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=16"],
    "rope_append.hip": ["-ffp-contract=off", "-mllvm", "-amdgpu-kernarg-preload-count=16"],
}

# the probes get the decode kernels' kernel-argument preloading, so that they
# are timed on the same footing
PROBE_FLAGS = ["-mllvm", "-amdgpu-kernarg-preload-count=16"]

COMMON_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-fPIC",
    "-std=c++17",
    "-Wall",
    # packed-FP32 VALU ops stay disabled in every kernel
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
]


def _hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    if cand.exists():
        return str(cand)
    found = shutil.which("hipcc")
    if not found:
        raise RuntimeError("hipcc not found (set ROCM_PATH)")
    return found


def build_library(verbose: bool = False) -> Path:
    """Compile every source and link the shared library; returns its path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    objects = []
    for name, extra in SOURCES.items():
        src = CSRC / name
        obj = BUILD_DIR / (src.stem + ".o")
        cmd = [hipcc, *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)]
        _run(cmd, verbose)
        objects.append(str(obj))
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    build_probe_library(verbose)
    return LIB_PATH


def build_probe_library(verbose: bool = False) -> Path:
    """Compile ``libflashdec_probe.so`` (bench.py's floor probes); returns its path."""
    tmp = PROBE_LIB_PATH.with_suffix(".so.tmp")
    _run([_hipcc(), *COMMON_FLAGS, *PROBE_FLAGS, "-shared", str(CSRC / PROBE_SOURCE), "-o", str(tmp)], verbose)
    os.replace(tmp, PROBE_LIB_PATH)
    return PROBE_LIB_PATH


def _run(cmd, verbose):
    if verbose:
        print(" ".join(cmd), flush=True)
    proc = subprocess.run(cmd, capture_output=True, text=True)
    # hipcc's host pass warns that it does not know the packed-fp32 feature
    noise = "is not a recognized feature for this target"
    err = "\n".join(line for line in proc.stderr.splitlines() if noise not in line)
    if proc.returncode != 0:
        raise RuntimeError(f"command failed ({proc.returncode}): {' '.join(cmd)}\n{err}")
    if verbose and err.strip():
        print(err)


if __name__ == "__main__":
    print(build_library(verbose=True))
