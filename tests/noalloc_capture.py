"""Run by test_zz_no_alloc.py in a process of its own, so that the first
vx_q8_linear_noalloc call on the GPU (the one that looks up the static
array's address) happens under HIP graph capture: the product is captured,
the graph replayed three times with eager work and synchronizations in
between, and every replay compared bit for bit with vx_q8_linear on a
scratch of VX_PREFILL_SPLIT_FLOATS partial sums. Prints "capture ok"."""
import ctypes
import pathlib
import sys

ROOT = pathlib.Path(__file__).resolve().parents[1]
sys.path.insert(0, str(ROOT))

import numpy as np  # noqa: E402
import torch  # noqa: E402

from voxcpm_amd import _lib, ops, synth  # noqa: E402


def main() -> int:
    device = torch.device("cuda:0")
    m, k, n = 320, 6144, 2048  # the tiled plan splits k four ways here
    rng = synth.Rng(202, m + n)
    blocks = synth.q8_blocks(rng, n, k)
    packed = ops.q8_pack(torch.from_numpy(blocks).to(device), n, k)
    x = torch.from_numpy(synth.activations(rng, m, k).view(np.int16)).to(device).view(
        torch.bfloat16)
    scratch = ops.Scratch(128, 1536)  # VX_PREFILL_SPLIT_FLOATS partial sums
    plan = (ctypes.c_int32 * 4)()
    _lib.check(_lib.lib().vx_q8_prefill_plan(m, k, n, scratch.handle, plan))
    assert plan[3] > 1, f"expected a split plan, got {list(plan)}"
    want = ops.q8_linear(x, packed, n, scratch=scratch)
    torch.cuda.synchronize()
    got = torch.full((m, n), float("nan"), dtype=torch.float32, device=device)
    capture = torch.cuda.Stream(device=device)
    graph = torch.cuda.CUDAGraph()
    print("capturing the first vx_q8_linear_noalloc call", flush=True)
    with torch.cuda.graph(graph, stream=capture):
        _lib.check(_lib.lib().vx_q8_linear_noalloc(
            x.data_ptr(), packed.data_ptr(), got.data_ptr(), m, k, n, 0,
            torch.cuda.current_stream().cuda_stream))
    for replay in range(3):
        got.fill_(float("nan"))
        # Eager work between replays: another product and a synchronization.
        ops.q8_linear(x, packed, n, scratch=scratch)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"replay {replay} differs from vx_q8_linear"
        print(f"replay {replay}: equal", flush=True)
    print("capture ok", flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
