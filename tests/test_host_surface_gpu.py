"""The C++ host surface (tests/cpp/host_test.cpp: Bf16Gemm::Linear,
DitSampler::Velocity and DitSampler::Sample over the C ABI) against the oracle.
The binary is built by __graft_entry__.build(); exit status 77 means no GPU."""
import pathlib
import subprocess

import pytest

pytestmark = pytest.mark.gpu

BINARY = pathlib.Path(__file__).resolve().parent / "cpp" / "bin" / "host_test"


def test_host_surface(cuda):
    assert BINARY.exists(), "build tests/cpp (python -c 'import __graft_entry__ as g; g.build()')"
    result = subprocess.run([str(BINARY)], capture_output=True, text=True, timeout=240)
    print(result.stdout)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "all host-surface checks match" in result.stdout
