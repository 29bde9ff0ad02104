"""Build ``liblvamd_hip.so`` for gfx950 with hipcc (no CMake, no torch headers),
and the native host planner ``_lvamd_host`` with g++.

Each HIP source compiles to an object in parallel; the objects link into one
shared library next to this file, which travels with the source tree.  The
host planner is a CPython extension module built against this interpreter's
headers, also next to this file.
Usage: ``python light-vllm_amd/build.py`` or ``__graft_entry__.build()``.
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
import sysconfig
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_ROOT = PACKAGE_DIR.parent
CSRC = PACKAGE_DIR / "csrc"
BUILD_DIR = PACKAGE_DIR / "_build"
LIB = PACKAGE_DIR / "liblvamd_hip.so"
ARCH = "gfx950"

HIPCC_FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++20",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    # Packed-FP32 VALU forms are disabled (plain float code only).
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    # Leading scalar kernel arguments (up to 16 dwords) arrive preloaded in
    # SGPRs, so a kernel's first address does not wait for an argument load.
    "-mllvm", "-amdgpu-kernarg-preload-count=16",
    f"-I{REPO_ROOT / 'include'}",
    f"-I{CSRC}",
]


def hipcc() -> str:
    found = shutil.which("hipcc") or "/opt/rocm/bin/hipcc"
    if not Path(found).exists():
        raise RuntimeError("hipcc not found (ROCm is required to build the HIP library)")
    return found


def _compile(src: Path) -> Path:
    obj = BUILD_DIR / (src.stem + ".o")
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    noise = "is not a recognized feature for this target"
    errors = "\n".join(l for l in proc.stderr.splitlines() if noise not in l)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{errors}")
    if errors.strip():
        print(errors, file=sys.stderr)
    return obj


HOST_SOURCE = CSRC / "lvamd_host.cpp"


def host_module_path() -> Path:
    """The native host planner, a CPython extension next to this file."""

    return PACKAGE_DIR / ("_lvamd_host" + sysconfig.get_config_var("EXT_SUFFIX"))


def _build_host() -> Path:
    """Compile the host planner with g++ against this interpreter's headers."""

    out = host_module_path()
    tmp = out.with_name(out.name + ".tmp")
    cxx = shutil.which("g++") or "g++"
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", "-Wextra", "-Wno-missing-field-initializers",
           f"-I{sysconfig.get_paths()['include']}", str(HOST_SOURCE), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed for {HOST_SOURCE.name}:\n{proc.stderr}")
    if proc.stderr.strip():
        print(proc.stderr, file=sys.stderr)
    os.replace(tmp, out)
    return out


def build(verbose: bool = True) -> Path:
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC.glob("*.hip"))
    jobs = min(len(sources) + 1, max(1, min(8, os.cpu_count() or 1)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        host = pool.submit(_build_host)
        objects = list(pool.map(_compile, sources))
        host.result()
    tmp = LIB.with_suffix(".so.tmp")
    cmd = [hipcc(), f"--offload-arch={ARCH}", "-shared", "-fPIC", "-o", str(tmp), *map(str, objects),
           "-Wl,-rpath,/opt/rocm/lib"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"link failed:\n{proc.stderr}")
    os.replace(tmp, LIB)
    if verbose:
        print(f"built {LIB} from {len(sources)} sources")
    return LIB


if __name__ == "__main__":
    build()
