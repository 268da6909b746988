"""vx_q8_linear_noalloc (the product for callers that cannot allocate: its
split partial sums live in a static device array) against vx_q8_linear
with a caller's scratch: bit for bit on two calls in a row, the second
smaller, each also within the reference's 1e-4 of the expanded arithmetic
in double (products_test.cpp:279-310); a skinny call (m <= 128) delegates
to the split-free plan."""
import ctypes
import pathlib
import sys

import numpy as np
import pytest
import torch

from voxcpm_amd import _lib, synth

pytestmark = pytest.mark.gpu


def noalloc():
    """The entry point through the C ABI (its ctypes signature is declared
    with the library's others)."""
    return _lib.lib().vx_q8_linear_noalloc


def expanded_error(y, x, blocks, oracle):
    m, k = x.shape
    n = y.shape[1]
    w = synth.bf16_values(oracle.q8_dequant_bf16(blocks, n, k)).astype(np.float64)
    xf = synth.bf16_values(x).astype(np.float64)
    magnitude = np.abs(xf) @ np.abs(w).T
    return float(np.max(np.abs(y - xf @ w.T) / np.maximum(magnitude, 1e-30)))


def test_noalloc_product_matches_scratch_product(vx, oracle, cuda, stream):
    function = noalloc()
    scratch = vx.Scratch(128, 16384)
    stream_handle = torch.cuda.current_stream().cuda_stream
    # Both tiled calls split k (4 splits of 80 tiles of 64 x 128).
    for m, k, n in [(320, 6144, 2048), (300, 6144, 2048), (22, 1024, 4096)]:
        print(f"noalloc product m={m} k={k} n={n}", flush=True)
        if m > 128:
            plan = (ctypes.c_int32 * 4)()
            _lib.check(_lib.lib().vx_q8_prefill_plan(m, k, n, scratch.handle, plan))
            assert plan[0] == 0 and plan[3] > 1, f"expected a split tiled plan: {list(plan)}"
        rng = synth.Rng(101, m + n)
        blocks = synth.q8_blocks(rng, n, k)
        packed = vx.q8_pack(torch.from_numpy(blocks).to(cuda), n, k)
        x_host = synth.activations(rng, m, k)
        x = torch.from_numpy(x_host.view(np.int16)).to(cuda).view(torch.bfloat16)
        want = vx.q8_linear(x, packed, n, scratch=scratch)
        got = torch.full((m, n), float("nan"), dtype=torch.float32, device=cuda)
        _lib.check(function(x.data_ptr(), packed.data_ptr(), got.data_ptr(), m, k, n, 0,
                            stream_handle))
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"m={m}: differs from vx_q8_linear"
        if m > 128:
            assert expanded_error(got.cpu().numpy(), x_host, blocks, oracle) <= 1e-4
        else:
            assert oracle.q8_check(got.cpu().numpy(), x_host, blocks) <= 1e-5


def test_noalloc_first_call_under_graph_capture(cuda):
    """The advertised use: the first call on a GPU (which looks up the
    static array's address) happens under HIP graph capture, and every
    replay equals vx_q8_linear bit for bit (tests/noalloc_capture.py, in a
    process of its own so that no earlier call has looked the address up)."""
    import subprocess
    script = pathlib.Path(__file__).resolve().parent / "noalloc_capture.py"
    result = subprocess.run([sys.executable, "-u", str(script)], capture_output=True, text=True,
                            timeout=180)
    print(result.stdout)
    assert result.returncode == 0, result.stdout + result.stderr
    assert "capture ok" in result.stdout
