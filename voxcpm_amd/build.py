"""Builds the voxcpm_amd library for gfx950 in-tree.

    python -m voxcpm_amd.build        # or voxcpm_amd.build.build()

Compiles every csrc/*.hip (the kernels and the C ABI) and host/*.cpp (the
C++ operator surface over the C ABI) with hipcc, objects under _build/, and
links voxcpm_amd/libvoxcpm_amd.so. Always rebuilds.
"""
from __future__ import annotations

import concurrent.futures
import os
import pathlib
import subprocess
import sys

PACKAGE = pathlib.Path(__file__).resolve().parent
ROOT = PACKAGE.parent
CSRC = PACKAGE / "csrc"
HOST = PACKAGE / "host"
BUILD = ROOT / "_build" / "voxcpm_amd"
LIBRARY = PACKAGE / "libvoxcpm_amd.so"
ARCH = "gfx950"

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    f"--offload-arch={ARCH}",
    "-O3",
    "-std=c++17",
    "-fPIC",
    "-Wall",
    # Packed float32 instructions stay off: the compiler forms them from
    # ordinary float code otherwise.
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{ROOT / 'include'}",
    f"-I{CSRC}",
]


def sources() -> list[pathlib.Path]:
    return sorted(CSRC.glob("*.hip")) + sorted(HOST.glob("*.cpp"))


def _compile(source: pathlib.Path) -> pathlib.Path:
    obj = BUILD / (source.parent.name + "_" + source.stem + ".o")
    cmd = [HIPCC, *FLAGS, "-c", str(source), "-o", str(obj)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"hipcc failed on {source.name}:\n{result.stderr}")
    return obj


def build(jobs: int | None = None, verbose: bool = False) -> pathlib.Path:
    BUILD.mkdir(parents=True, exist_ok=True)
    srcs = sources()
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        objects = list(pool.map(_compile, srcs))
    tmp = LIBRARY.with_suffix(".so.tmp")
    cmd = [HIPCC, f"--offload-arch={ARCH}", "-shared", "-o", str(tmp),
           *map(str, objects)]
    result = subprocess.run(cmd, capture_output=True, text=True)
    if result.returncode != 0:
        raise RuntimeError(f"link failed:\n{result.stderr}")
    os.replace(tmp, LIBRARY)
    if verbose:
        print(f"built {LIBRARY}")
    return LIBRARY


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
