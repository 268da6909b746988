"""Every kernel of the library keeps its values in registers: the compiler's
resource remarks (a device-only compile of each csrc/*.hip for gfx950, no
GPU needed) report no scratch memory, so no kernel spills registers to
memory. A kernel that spills pays a memory round trip per spilled value on
its critical path."""
import pytest

from voxcpm_amd import build


@pytest.fixture(scope="module")
def report():
    return build.resource_report()


def test_kernels_found(report):
    # The product engine, the DiT's fused kernels and the persistent
    # evaluation are all in the report.
    names = " ".join(report)
    for part in ("EngineKernel", "AttentionKernel", "EvaluateKernel", "GemmKernel",
                 "TiledKernel"):
        assert part in names, part


def test_no_kernel_uses_scratch(report):
    spilling = {name: r for name, r in report.items() if r.get("scratch", 0) > 0}
    assert not spilling, spilling


def test_register_budget(report):
    # At most 256 VGPRs per lane (gfx950's architectural limit for one wave);
    # the 1024-thread kernels fit 128 (every SIMD holds four waves).
    for name, r in report.items():
        assert r.get("vgprs", 0) <= 256, (name, r)
