"""The stack with a key/value cache (vx_stack: VoxCPM2's base and residual
LMs and the local encoder) and its split-key attention on the GPU against
the CPU oracle, on identical seeded inputs.

Tolerances (fp32 accumulation, bf16 activations, different summation
orders): attention outputs within one bf16 ulp of the oracle's (a rounding
boundary may fall differently after float32 reassociation); stack outputs,
residual streams and caches max |gpu - oracle| / max |oracle| <= 1e-2 and
cosine >= 0.9999 -- the bound the DiT's parity states -- while the measured
errors are reported far below it.
"""
import numpy as np
import pytest
import torch

from voxcpm_amd import _lib, synth
from test_dit_gpu import cosine, dev, host_bf16, rel_max, ulp_diff

pytestmark = pytest.mark.gpu

BOUND = 1e-2
COSINE = 0.9999


def f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


@pytest.mark.parametrize("heads,kv_heads,head_dim", [(16, 2, 128), (4, 4, 64), (8, 1, 128)])
@pytest.mark.parametrize("rows,rps,past,causal", [
    (1, 1, 0, True),      # the first decode step: one key
    (1, 1, 63, True),     # one chunk exactly
    (1, 1, 64, True),     # two chunks, the second of one key
    (1, 1, 700, True),    # eleven chunks merged
    (1, 1, 4200, True),   # 66 chunks: the merge's second pass over chunks 64..
    (1, 1, 8300, True),   # 130 chunks: more than two passes of the merge
    (3, 3, 130, True),    # causal rows of one sequence beyond a chunk
    (10, 5, 0, False),    # the encoder: two 5-row sequences, bidirectional
])
def test_split_attention_against_oracle(vx, oracle, cuda, stream, heads, kv_heads, head_dim,
                                        rows, rps, past, causal):
    rng = synth.Rng(31, rows * 1000 + past + head_dim)
    sequences = rows // rps
    keys = past + rps
    capacity = (sequences - 1) * keys + keys + 3
    q = f32(rng.normal(rows * heads * head_dim).reshape(rows, heads, head_dim))
    kc = f32(rng.normal(kv_heads * capacity * head_dim).reshape(kv_heads, capacity, head_dim))
    vc = f32(rng.normal(kv_heads * capacity * head_dim).reshape(kv_heads, capacity, head_dim))
    ref = np.zeros((rows, heads, head_dim), np.uint16)
    oracle.lib().vo_attention(oracle.ptr(q), oracle.ptr(kc), oracle.ptr(vc), oracle.ptr(ref),
                              rows, rps, keys, past, int(causal), heads, kv_heads, head_dim,
                              capacity)
    got = vx.split_attention(dev(q, cuda), dev(kc, cuda), dev(vc, cuda), rps, keys, past,
                             causal, heads, kv_heads)
    torch.cuda.synchronize()
    diff = ulp_diff(host_bf16(got), ref)
    assert diff.max() <= 1, f"max {diff.max()} ulp"


def make_stack(vx, oracle, config, seed, bf16_weights=False, positions=2048):
    """`positions`: rows of the rotary table; every position a step uses
    must index it (the kernels read row `position` of the table)."""
    rope = None
    if config.rope:
        rope = oracle.rope_table(config.rope_theta, config.head_dim, config.rope_factors,
                                 config.rope_scaling, positions)
    weights = synth.stack_weights(config, seed)
    return (vx.Stack(weights, rope, bf16_weights=bf16_weights),
            oracle.OracleStack(weights, rope, threads=16, bf16_weights=bf16_weights))


def check_close(got, ref, what):
    error, cos = rel_max(got, ref), cosine(got, ref)
    print(f"{what}: rel max {error:.2e}, cosine {cos:.7f}", flush=True)
    assert error <= BOUND and cos >= COSINE, what


class Run:
    """One stack on the GPU and in the oracle with the same cache history."""

    def __init__(self, vx, oracle, cuda, config, seed, capacity, bf16_weights=False):
        # Positions here are cache rows, so a table of `capacity` rows
        # covers every step.
        self.gpu, self.cpu = make_stack(vx, oracle, config, seed, bf16_weights,
                                        positions=max(2048, capacity))
        self.config = config
        self.k_gpu, self.v_gpu = self.gpu.cache(capacity)
        shape = (config.layers, config.kv_heads, capacity, config.head_dim)
        self.k_cpu, self.v_cpu = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
        self.cuda = cuda

    def step(self, h0, positions, cache_rows, rps, kps, past, causal, what):
        positions = np.asarray(positions, np.int32)
        cache_rows = np.asarray(cache_rows, np.int32)
        hidden = dev(f32(h0), self.cuda)
        output = torch.empty_like(hidden)
        self.gpu.forward(hidden, output, dev(positions, self.cuda), dev(cache_rows, self.cuda),
                         rps, kps, past, causal, self.k_gpu, self.v_gpu)
        torch.cuda.synchronize()
        ref_h, ref_out = self.cpu.forward(h0, positions, cache_rows, rps, kps, past, causal,
                                          self.k_cpu, self.v_cpu)
        check_close(output.cpu().numpy(), ref_out, f"{what} output")
        check_close(hidden.cpu().numpy(), ref_h, f"{what} hidden")
        return output


STACKS = {
    "gqa-hd64": synth.StackConfig(hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512,
                                  layers=2),
    "no-rope-hd128": synth.StackConfig(hidden=512, heads=4, kv_heads=1, head_dim=128,
                                       ffn=1024, layers=2, rope=False),
    "voxcpm2-lm-2layers": synth.StackConfig(layers=2, rope_factors=synth.VOXCPM2_SHORT_FACTORS),
}


PATHS = {"auto": (_lib.STACK_PATH_AUTO, _lib.STACK_PATH_ROWS),
         "fragments": (_lib.STACK_PATH_FUSED, _lib.STACK_PATH_FUSED),
         "unfused": (_lib.STACK_PATH_UNFUSED, _lib.STACK_PATH_UNFUSED)}


@pytest.mark.parametrize("name", list(STACKS))
@pytest.mark.parametrize("path", list(PATHS))
def test_stack_prefill_then_decode(vx, oracle, cuda, stream, name, path):
    """A causal prefill of 7 rows, then one-row decode steps (positions =
    cache rows = past) through a cache long enough to split the attention
    into several chunks; the caches match too. AUTO takes the one-tile
    row-major kernels at these row counts."""
    config = STACKS[name]
    run = Run(vx, oracle, cuda, config, 41, capacity=160)
    selected, expected = PATHS[path]
    run.gpu.set_path(selected)
    assert run.gpu.path(1) == expected
    rng = synth.Rng(42, 1)
    prefix = 7
    h0 = rng.normal(prefix * config.hidden).astype(np.float32).reshape(prefix, config.hidden)
    rows = np.arange(prefix)
    run.step(h0, rows, rows, prefix, prefix, 0, True, f"{name} prefill")
    # Jump the history to 120 cached positions (the oracle's and the
    # GPU's caches filled alike), then decode three steps past two chunks.
    filler = rng.normal(2 * config.layers * config.kv_heads * 113 * config.head_dim)
    filler = f32(filler).reshape(2, config.layers, config.kv_heads, 113, config.head_dim)
    run.k_cpu[:, :, prefix:120] = filler[0]
    run.v_cpu[:, :, prefix:120] = filler[1]
    run.k_gpu[:, :, prefix:120] = torch.from_numpy(filler[0]).to(cuda)
    run.v_gpu[:, :, prefix:120] = torch.from_numpy(filler[1]).to(cuda)
    for position in (120, 121, 122):
        h = rng.normal(config.hidden).astype(np.float32).reshape(1, config.hidden)
        run.step(h, [position], [position], 1, 1, position, True, f"{name} decode {position}")
    check_close(run.k_gpu.cpu().numpy(), run.k_cpu, f"{name} key cache")
    check_close(run.v_gpu.cpu().numpy(), run.v_cpu, f"{name} value cache")


def test_stack_encoder_layout(vx, oracle, cuda, stream):
    """The local encoder's call (generator.cpp:252-295): patches of 5 rows
    attending within themselves, rotary positions row % 5, cache rows in
    order; three and four patches at once (15 and 20 rows: the
    fragment-order kernels) and one alone (the one-tile kernels)."""
    config = synth.StackConfig(hidden=1024, ffn=4096, layers=2,
                               rope_factors=synth.VOXCPM2_SHORT_FACTORS)
    run = Run(vx, oracle, cuda, config, 43, capacity=64)
    rng = synth.Rng(44, 1)
    for patches in (3, 4, 1):
        rows = 5 * patches
        expected = _lib.STACK_PATH_ROWS if rows <= 8 else _lib.STACK_PATH_FUSED
        assert run.gpu.path(rows) == expected
        h0 = rng.normal(rows * config.hidden).astype(np.float32).reshape(rows, config.hidden)
        run.step(h0, np.arange(rows) % 5, np.arange(rows), 5, 5, 0, False,
                 f"encoder {patches} patches")


def test_stack_many_rows_unfused(vx, oracle, cuda, stream):
    """More rows than the fused kernels take (a 40-row causal prefill)
    run the reference's launch sequence."""
    config = STACKS["gqa-hd64"]
    run = Run(vx, oracle, cuda, config, 45, capacity=48)
    assert run.gpu.path(40) == _lib.STACK_PATH_UNFUSED
    rng = synth.Rng(46, 1)
    h0 = rng.normal(40 * config.hidden).astype(np.float32).reshape(40, config.hidden)
    rows = np.arange(40)
    run.step(h0, rows, rows, 40, 40, 0, True, "prefill 40")


def test_stack_bf16_weights(vx, oracle, cuda, stream):
    config = STACKS["gqa-hd64"]
    run = Run(vx, oracle, cuda, config, 47, capacity=80, bf16_weights=True)
    rng = synth.Rng(48, 1)
    h0 = rng.normal(5 * config.hidden).astype(np.float32).reshape(5, config.hidden)
    rows = np.arange(5)
    run.step(h0, rows, rows, 5, 5, 0, True, "bf16 prefill")
    h = rng.normal(config.hidden).astype(np.float32).reshape(1, config.hidden)
    run.step(h, [5], [5], 1, 1, 5, True, "bf16 decode")


def test_stack_argument_errors(vx, cuda, stream):
    """Bad layouts fail before anything is launched."""
    config = STACKS["gqa-hd64"]
    weights = synth.stack_weights(config, 49)
    rope = np.zeros((64, config.head_dim), np.float32)
    stack = vx.Stack(weights, rope)
    k, v = stack.cache(16)
    hidden = torch.zeros((4, config.hidden), dtype=torch.float32, device=cuda)
    out = torch.empty_like(hidden)
    rows = torch.arange(4, dtype=torch.int32, device=cuda)
    with pytest.raises(_lib.VxError) as info:  # rows not a multiple of rows_per_sequence
        stack.forward(hidden, out, rows, rows, 3, 3, 0, True, k, v)
    assert info.value.status == _lib.VX_BAD_ARG
    with pytest.raises(_lib.VxError) as info:  # keys past the capacity
        stack.forward(hidden, out, rows, rows, 4, 4, 13, True, k, v)
    assert info.value.status == _lib.VX_BAD_ARG
    with pytest.raises(_lib.VxError) as info:  # two sequences 10 keys apart
        stack.forward(hidden, out, rows, rows, 2, 10, 5, False, k, v)
    assert info.value.status == _lib.VX_BAD_ARG


def test_stack_decode_replays(vx, oracle, cuda, stream):
    """Decode steps through the same buffers replay one captured graph
    whose attention reads each call's past from the device: every step
    matches the oracle, across chunk boundaries (63 -> 64 -> 65 keys), and a
    per-kernel call and a fragment-order call in between (other paths, the
    graph dropped and captured again) change nothing."""
    config = STACKS["gqa-hd64"]
    run = Run(vx, oracle, cuda, config, 51, capacity=200)
    rng = synth.Rng(52, 1)
    hidden = torch.empty((1, config.hidden), dtype=torch.float32, device=cuda)
    output = torch.empty_like(hidden)
    position = torch.empty(1, dtype=torch.int32, device=cuda)
    for past in (61, 62, 63, 64, 65, 129, 130):
        h = rng.normal(config.hidden).astype(np.float32).reshape(1, config.hidden)
        hidden.copy_(torch.from_numpy(h))
        position.fill_(past)
        run.gpu.set_path(_lib.STACK_PATH_UNFUSED if past == 64 else
                         _lib.STACK_PATH_FUSED if past == 129 else _lib.STACK_PATH_AUTO)
        run.gpu.forward(hidden, output, position, position, 1, 1, past, True, run.k_gpu,
                        run.v_gpu)
        torch.cuda.synchronize()
        at = np.array([past], np.int32)
        ref_h, ref_out = run.cpu.forward(h, at, at, 1, 1, past, True, run.k_cpu, run.v_cpu)
        check_close(output.cpu().numpy(), ref_out, f"replay past {past} output")
        check_close(hidden.cpu().numpy(), ref_h, f"replay past {past} hidden")


def test_stack_decode_key_bands(vx, oracle, cuda, stream):
    """Replayed decode steps keep one graph per 256-key band of attended
    keys: steps across band edges (255 -> 256 -> 257 keys, 512 -> 513),
    back into an earlier band (its graph replayed again) and forward again
    all match the oracle."""
    config = STACKS["gqa-hd64"]
    run = Run(vx, oracle, cuda, config, 55, capacity=700)
    rng = synth.Rng(56, 1)
    hidden = torch.empty((1, config.hidden), dtype=torch.float32, device=cuda)
    output = torch.empty_like(hidden)
    position = torch.empty(1, dtype=torch.int32, device=cuda)
    run.gpu.set_path(_lib.STACK_PATH_AUTO)
    for past in (10, 254, 255, 256, 300, 511, 512, 100, 513, 698):
        h = rng.normal(config.hidden).astype(np.float32).reshape(1, config.hidden)
        hidden.copy_(torch.from_numpy(h))
        position.fill_(past)
        run.gpu.forward(hidden, output, position, position, 1, 1, past, True, run.k_gpu,
                        run.v_gpu)
        torch.cuda.synchronize()
        at = np.array([past], np.int32)
        ref_h, ref_out = run.cpu.forward(h, at, at, 1, 1, past, True, run.k_cpu, run.v_cpu)
        check_close(output.cpu().numpy(), ref_out, f"band past {past} output")
        check_close(hidden.cpu().numpy(), ref_h, f"band past {past} hidden")


def test_stack_decode_replays_past_4096(vx, oracle, cuda, stream):
    """The base LM's long-context decode (4096 cached positions and more:
    65 and more 64-key chunks, so the chunk merge takes its later passes)
    replayed from one captured graph, every step against the oracle, over a
    cache filled with random keys and values."""
    config = STACKS["gqa-hd64"]
    capacity = 4300
    run = Run(vx, oracle, cuda, config, 53, capacity=capacity)
    rng = synth.Rng(54, 1)
    filled = 4094
    filler = rng.normal(2 * config.layers * config.kv_heads * filled * config.head_dim)
    filler = f32(filler).reshape(2, config.layers, config.kv_heads, filled, config.head_dim)
    run.k_cpu[:, :, :filled] = filler[0]
    run.v_cpu[:, :, :filled] = filler[1]
    run.k_gpu[:, :, :filled] = torch.from_numpy(filler[0]).to(cuda)
    run.v_gpu[:, :, :filled] = torch.from_numpy(filler[1]).to(cuda)
    hidden = torch.empty((1, config.hidden), dtype=torch.float32, device=cuda)
    output = torch.empty_like(hidden)
    position = torch.empty(1, dtype=torch.int32, device=cuda)
    run.gpu.set_path(_lib.STACK_PATH_AUTO)
    for past in range(filled, filled + 8):  # 4095 .. 4102 keys: 64 -> 65 chunks
        assert past < capacity  # the position indexes the cache and the rotary table
        h = rng.normal(config.hidden).astype(np.float32).reshape(1, config.hidden)
        hidden.copy_(torch.from_numpy(h))
        position.fill_(past)
        run.gpu.forward(hidden, output, position, position, 1, 1, past, True, run.k_gpu,
                        run.v_gpu)
        torch.cuda.synchronize()
        at = np.array([past], np.int32)
        ref_h, ref_out = run.cpu.forward(h, at, at, 1, 1, past, True, run.k_cpu, run.v_cpu)
        check_close(output.cpu().numpy(), ref_out, f"replay past {past} output")
        check_close(hidden.cpu().numpy(), ref_h, f"replay past {past} hidden")
