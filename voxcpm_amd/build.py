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


def resource_report(jobs: int | None = None) -> dict[str, dict[str, int]]:
    """Compiles every csrc/*.hip for the device only with the compiler's
    kernel resource remarks and returns {kernel symbol: {"vgprs", "sgprs",
    "scratch", "vgpr_spill", "sgpr_spill"}} (scratch in bytes per lane)."""
    import re
    import tempfile
    fields = {"VGPRs": "vgprs", "TotalSGPRs": "sgprs", "ScratchSize [bytes/lane]": "scratch",
              "VGPRs Spill": "vgpr_spill", "SGPRs Spill": "sgpr_spill"}

    def remarks(source: pathlib.Path) -> dict[str, dict[str, int]]:
        with tempfile.TemporaryDirectory() as tmp:
            cmd = [HIPCC, *FLAGS, "--cuda-device-only", "-Rpass-analysis=kernel-resource-usage",
                   "-c", str(source), "-o", str(pathlib.Path(tmp) / "device.o")]
            result = subprocess.run(cmd, capture_output=True, text=True)
        if result.returncode != 0:
            raise RuntimeError(f"hipcc failed on {source.name}:\n{result.stderr}")
        kernels: dict[str, dict[str, int]] = {}
        current = None
        for line in result.stderr.splitlines():
            match = re.search(r"remark: +Function Name: (\S+)", line)
            if match:
                current = kernels.setdefault(match.group(1), {})
                continue
            for label, key in fields.items():
                match = re.search(r"remark: +" + re.escape(label) + r": (\d+)", line)
                if match and current is not None:
                    current[key] = int(match.group(1))
        return kernels

    srcs = sorted(CSRC.glob("*.hip"))
    jobs = jobs or min(len(srcs), os.cpu_count() or 4, 8)
    report: dict[str, dict[str, int]] = {}
    with concurrent.futures.ThreadPoolExecutor(jobs) as pool:
        for kernels in pool.map(remarks, srcs):
            report.update(kernels)
    return report


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
