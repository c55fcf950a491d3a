"""Compile the HIP kernels under ``csrc/`` into ``libcdb_amd.so`` for gfx950, and the
host tick core ``csrc/tick.cpp`` into the ``_tick`` extension module.

The library is built in-tree next to this file so that it travels with the
source tree; object files go to ``_build/`` at the repository root. Every call
recompiles (objects are rebuilt only when their source or a header changed).
"""

from __future__ import annotations

import os
import shutil
import subprocess
import sysconfig
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PACKAGE_DIR = Path(__file__).resolve().parent
REPO_DIR = PACKAGE_DIR.parent
CSRC_DIR = PACKAGE_DIR / "csrc"
INCLUDE_DIR = REPO_DIR / "include"
BUILD_DIR = REPO_DIR / "_build"
LIBRARY_PATH = PACKAGE_DIR / "libcdb_amd.so"
OFFLOAD_ARCH = "gfx950"

# Packed-fp32 VALU forms are kept out of the generated code; hipcc's host pass
# reports the feature as unknown, which is harmless.
HIP_FLAGS = [
    f"--offload-arch={OFFLOAD_ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Xclang",
    "-target-feature",
    "-Xclang",
    "-packed-fp32-ops",
    f"-I{INCLUDE_DIR}",
]


# Per-source additions. The prefill kernel keeps its MFMA accumulators in
# ordinary VGPRs: its online softmax rescales them between products, which in
# the accumulator-register form costs a move out and back for every element.
FILE_FLAGS = {
    "prefill_attention.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}


def _hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found; the CDB kernels need the ROCm HIP compiler")


def _headers() -> list[Path]:
    return sorted(CSRC_DIR.glob("*.h")) + sorted(INCLUDE_DIR.glob("*.h"))


def _needs_rebuild(obj: Path, src: Path, headers: list[Path]) -> bool:
    if not obj.exists():
        return True
    obj_mtime = obj.stat().st_mtime
    return any(dep.stat().st_mtime > obj_mtime for dep in (src, *headers, Path(__file__)))


def _compile(hipcc: str, src: Path, obj: Path) -> None:
    cmd = [hipcc, *HIP_FLAGS, *FILE_FLAGS.get(src.name, []), "-c", str(src), "-o", str(obj)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{proc.stderr}")


def build_library(*, force: bool = False, jobs: int | None = None) -> Path:
    """Compile every ``csrc/*.hip`` source and link ``libcdb_amd.so``; return its path."""

    hipcc = _hipcc()
    BUILD_DIR.mkdir(exist_ok=True)
    sources = sorted(CSRC_DIR.glob("*.hip"))
    if not sources:
        raise RuntimeError(f"no HIP sources under {CSRC_DIR}")
    headers = _headers()
    objects = [BUILD_DIR / (src.stem + ".o") for src in sources]
    stale = [(src, obj) for src, obj in zip(sources, objects) if force or _needs_rebuild(obj, src, headers)]
    workers = jobs or min(8, max(1, len(stale)))
    with ThreadPoolExecutor(max_workers=workers) as pool:
        list(pool.map(lambda pair: _compile(hipcc, *pair), stale))
    tmp = LIBRARY_PATH.with_suffix(".so.tmp")
    link = [hipcc, f"--offload-arch={OFFLOAD_ARCH}", "-shared", "-fPIC", *map(str, objects), "-o", str(tmp)]
    proc = subprocess.run(link, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"linking libcdb_amd.so failed:\n{proc.stderr}")
    os.replace(tmp, LIBRARY_PATH)
    return LIBRARY_PATH


TICK_SOURCE = CSRC_DIR / "tick.cpp"
TICK_PATH = PACKAGE_DIR / ("_tick" + (sysconfig.get_config_var("EXT_SUFFIX") or ".so"))


def build_tick(*, force: bool = False) -> Path:
    """Compile the host tick core (``csrc/tick.cpp``, a CPython extension) with g++."""

    if not force and TICK_PATH.exists() and TICK_PATH.stat().st_mtime >= TICK_SOURCE.stat().st_mtime:
        return TICK_PATH
    cxx = shutil.which(os.environ.get("CXX", "g++")) or shutil.which("g++")
    if not cxx:
        raise RuntimeError("g++ not found; the host tick core needs a C++ compiler")
    tmp = TICK_PATH.with_name(TICK_PATH.name + ".tmp")
    cmd = [cxx, "-O2", "-std=c++17", "-shared", "-fPIC", "-Wall", f"-I{sysconfig.get_paths()['include']}",
           str(TICK_SOURCE), "-o", str(tmp)]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    if proc.returncode != 0:
        raise RuntimeError(f"g++ failed for {TICK_SOURCE.name}:\n{proc.stderr}")
    os.replace(tmp, TICK_PATH)
    return TICK_PATH


def build_all(*, force: bool = False) -> tuple[Path, Path]:
    return build_library(force=force), build_tick(force=force)


if __name__ == "__main__":
    print(build_all())
