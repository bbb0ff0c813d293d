"""Build ``libflashdec_hip.so`` (the C-ABI library) in-tree with hipcc for gfx950,
``libflashdec_probe.so`` (bench.py's floor probes, ``csrc/floor_probe.hip``) and
``libflashdec_timeline.so`` (the same library with the decode kernel's per-wave
timeline stamps compiled in, ``-DFD_TIMELINE``; bench.py's c2-timeline
workload only).

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
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB_PATH = PACKAGE_DIR / "libflashdec_hip.so"
# measurement probes for bench.py's floor workload (not the decode library)
PROBE_SOURCE = "floor_probe.hip"
PROBE_LIB_PATH = PACKAGE_DIR / "libflashdec_probe.so"
# measurement build of the decode library (per-wave timeline stamps)
TIMELINE_LIB_PATH = PACKAGE_DIR / "libflashdec_timeline.so"
TIMELINE_SOURCE = "paged_decode.hip"
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
    """Compile every source and link the shared library (and the timeline and
    probe libraries beside it); returns the library's path."""
    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    objects, jobs = [], []
    for name, extra in SOURCES.items():
        src = CSRC / name
        obj = BUILD_DIR / (src.stem + ".o")
        jobs.append([hipcc, *COMMON_FLAGS, *extra, "-c", str(src), "-o", str(obj)])
        objects.append(str(obj))
    # the timeline build differs in the decode kernels' file only
    tl_obj = BUILD_DIR / "paged_decode_timeline.o"
    jobs.append([hipcc, *COMMON_FLAGS, *SOURCES[TIMELINE_SOURCE], "-DFD_TIMELINE", "-c", str(CSRC / TIMELINE_SOURCE),
                 "-o", str(tl_obj)])
    with ThreadPoolExecutor(max_workers=min(len(jobs), os.cpu_count() or 1)) as pool:
        for f in [pool.submit(_run, cmd, verbose) for cmd in jobs]:
            f.result()
    tmp = LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *objects, "-o", str(tmp)], verbose)
    os.replace(tmp, LIB_PATH)
    tl_objects = [str(tl_obj) if Path(o).stem == Path(TIMELINE_SOURCE).stem else o for o in objects]
    tmp = TIMELINE_LIB_PATH.with_suffix(".so.tmp")
    _run([hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *tl_objects, "-o", str(tmp)], verbose)
    os.replace(tmp, TIMELINE_LIB_PATH)
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
