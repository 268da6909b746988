"""Q8_0 panels and products on the GPU against the CPU oracle.

Mirrors the reference's tests/products_test.cpp: random GGML Q8_0 blocks
(q uniform in [-128, 127], float16 scale bits uniform in [0x1000, 0x1C00])
and bf16 activations ~ N(0, 2) at VoxCPM2's shapes and odd ones, every row
count up to 32, with and without accumulation and under several split
plans, each compared with a double-precision sum: the error relative to
sum |x w| of each output must stay <= 1e-5 (products_test.cpp:117-145,
229). The dequantization and the layout round trip are bit-exact.
"""
import numpy as np
import pytest
import torch

from voxcpm_amd import synth

pytestmark = pytest.mark.gpu

ALL_ROWS = [1, 2, 4, 5, 8, 11, 16, 22, 32]
# products_test.cpp:326-338 (k = in, n = out)
SHAPES = [
    (64, 1024, [4, 8]),
    (512, 1024, [1, 4]),
    (1024, 2560, ALL_ROWS),
    (2048, 1024, [1, 5, 22]),
    (4096, 1024, [1, 5, 22]),
    (2048, 2048, [1, 5]),
    (6144, 2048, [1, 3, 5]),
    # the LM decode step's qkv and gate_up (tools/bench/gemm_bench.cpp:35-36)
    (2048, 2560, [1, 5]),
    (2048, 12288, [1, 5]),
    (8192, 512, [1, 22]),
    (1024, 72, [3, 22]),  # rows not a multiple of 16
    (2048, 2, [1]),
    # odd block counts: the last pair's second block is past k
    (96, 40, [1, 9, 22, 32]),
    (160, 17, [3, 22]),
]
LIMIT = 1e-5


def reference_weights(rng: synth.Rng, n: int, k: int) -> np.ndarray:
    """products_test.cpp:65-86: q in [-128, 127], scale bits 0x1000..0x1C00."""
    count = n * (k // 32)
    blocks = np.empty((count, 34), dtype=np.uint8)
    bits = (0x1000 + (rng.bits(count) % np.uint64(0xC01))).astype(np.uint16)
    blocks[:, 0] = (bits & 0xFF).astype(np.uint8)
    blocks[:, 1] = (bits >> 8).astype(np.uint8)
    q = ((rng.bits(count * 32) % np.uint64(256)).astype(np.int64) - 128)
    blocks[:, 2:] = q.astype(np.int8).view(np.uint8).reshape(count, 32)
    return blocks.reshape(n, k // 32, 34)


def reference_activations(rng: synth.Rng, rows: int, k: int) -> np.ndarray:
    return synth.bf16_bits(rng.normal(rows * k, 2.0).astype(np.float32)).reshape(rows, k)


def to_device(array: np.ndarray, cuda) -> torch.Tensor:
    if array.dtype == np.uint16:
        return torch.from_numpy(array.view(np.int16).copy()).to(cuda).view(torch.bfloat16)
    return torch.from_numpy(np.ascontiguousarray(array)).to(cuda)


def bf16_host(tensor: torch.Tensor) -> np.ndarray:
    return tensor.view(torch.int16).cpu().numpy().view(np.uint16)


@pytest.mark.parametrize("k,n", [(s[0], s[1]) for s in SHAPES] + [(96, 40), (160, 17)])
def test_layout_round_trip_and_dequant(vx, oracle, cuda, stream, k, n):
    rng = synth.Rng(1234, k * 7 + n)
    blocks = reference_weights(rng, n, k)
    raw = to_device(blocks, cuda)
    packed = vx.q8_pack(raw, n, k)
    assert packed.numel() == ((n + 15) // 16) * ((k + 63) // 64) * 1088
    back = vx.q8_unpack_blocks(packed, n, k)
    dequant = vx.q8_unpack_bf16(packed, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(back.cpu().numpy(), blocks), "pack/unpack round trip"
    expected = oracle.q8_dequant_bf16(blocks, n, k)
    assert np.array_equal(bf16_host(dequant), expected), "bf16(scale * q)"


def test_dequant_special_values(vx, oracle, cuda, stream):
    """q = -128, +-0, subnormal, negative, infinite and NaN scales."""
    n, k = 16, 64
    rng = synth.Rng(5, 5)
    blocks = reference_weights(rng, n, k)
    scales = [0x0000, 0x8000, 0x0001, 0x03FF, 0x0400, 0x8001, 0x7BFF, 0xFBFF,
              0x7C00, 0xFC00, 0x7E00, 0x3C00, 0x1000, 0x1C00, 0x0200, 0x83FF]
    flat = blocks.reshape(-1, 34)
    for i in range(flat.shape[0]):
        bits = scales[i % len(scales)]
        flat[i, 0] = bits & 0xFF
        flat[i, 1] = bits >> 8
    flat[:, 2] = np.uint8(0x80)  # q = -128
    flat[:, 3] = np.uint8(0x7F)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    dequant = bf16_host(vx.q8_unpack_bf16(packed, n, k))
    expected = oracle.q8_dequant_bf16(blocks, n, k)
    assert np.array_equal(dequant, expected)


def run_product(vx, x_dev, packed, n, before, plan, scratch, cuda):
    m = x_dev.shape[0]
    y = torch.from_numpy(before.copy()).to(cuda) if before is not None else None
    out = vx.q8_linear(x_dev, packed, n, y=y, accumulate=before is not None,
                       scratch=scratch, plan=plan)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("k,n,rows_list", SHAPES)
def test_products_against_double(vx, oracle, cuda, stream, k, n, rows_list):
    rng = synth.Rng(1234, 10 * k + n)
    blocks = reference_weights(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    scratch = vx.Scratch(32, n)
    for rows in rows_list:
        x = reference_activations(rng, rows, k)
        x_dev = to_device(x, cuda)
        before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
        # Default plan, one workgroup per tile and wave, and forced splits
        # (the reference's PlanWmma targets 1, default and 4096 waves).
        plans = [None, (1, 1, 1), (1, 4, 1), (2, 2, 4), (1, 4, 8)]
        for accumulate in (False, True):
            results = []
            for plan in plans:
                y = run_product(vx, x_dev, packed, n,
                                before if accumulate else None, plan, scratch, cuda)
                worst = oracle.q8_check(y, x, blocks, before if accumulate else None)
                assert worst <= LIMIT, (
                    f"rows {rows} k {k} n {n} plan {plan} accumulate {accumulate}:"
                    f" worst {worst:.3e}")
                results.append(y)
            # The oracle's float32 arithmetic agrees to the same bound.
            ref = oracle.q8_linear(x, blocks, n, before if accumulate else None)
            assert oracle.q8_check(ref, x, blocks,
                                   before if accumulate else None) <= LIMIT
            scale = np.abs(ref).max() + 1e-30
            assert np.abs(results[0] - ref).max() / scale < 1e-4


def test_split_counters_reset(vx, oracle, cuda, stream):
    """A split product twice in a row: the second finds its counters at
    zero (the first reset them) and is bitwise equal to the first
    (products_test.cpp:241-251; determinism)."""
    k, n, rows = 4096, 1024, 22
    rng = synth.Rng(77, 1)
    blocks = reference_weights(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x = reference_activations(rng, rows, k)
    x_dev = to_device(x, cuda)
    scratch = vx.Scratch(32, n)
    first = run_product(vx, x_dev, packed, n, None, (1, 4, 8), scratch, cuda)
    second = run_product(vx, x_dev, packed, n, None, (1, 4, 8), scratch, cuda)
    assert np.array_equal(first, second)
    assert oracle.q8_check(second, x, blocks) <= LIMIT
    third = run_product(vx, x_dev, packed, n, None, None, scratch, cuda)
    fourth = run_product(vx, x_dev, packed, n, None, None, scratch, cuda)
    assert np.array_equal(third, fourth)


@pytest.mark.parametrize("rows", [17, 22, 32])
def test_forced_engine_plans(vx, oracle, cuda, stream, rows):
    """The engine with forced plans (vx_q8_linear_engine: row groups, waves,
    pairs per wave, row blocks), the plan search behind the default plans:
    every plan within 1e-5 of sum |x w| and equal to the default plan's
    result to float32 rounding."""
    from voxcpm_amd import _lib
    k, n = 2048, 1040  # 65 row groups: a ragged last workgroup for 2 and 4
    rng = synth.Rng(78, rows)
    blocks = reference_weights(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x = reference_activations(rng, rows, k)
    x_dev = to_device(x, cuda)
    default = run_product(vx, x_dev, packed, n, None, None, None, cuda)
    handle = torch.cuda.current_stream().cuda_stream
    for rg, waves, pw, blocks_ in [(1, 16, 1, 1), (2, 8, 2, 2), (4, 8, 1, 4), (1, 4, 2, 3),
                                   (2, 16, 2, 1), (4, 4, 1, 2)]:
        y = torch.full((rows, n), float("nan"), dtype=torch.float32, device=cuda)
        _lib.check(_lib.lib().vx_q8_linear_engine(x_dev.data_ptr(), packed.data_ptr(),
                                                  y.data_ptr(), rows, k, n, rg, waves, pw,
                                                  blocks_, handle))
        torch.cuda.synchronize()
        got = y.cpu().numpy()
        worst = oracle.q8_check(got, x, blocks)
        assert worst <= LIMIT, f"plan {(rg, waves, pw, blocks_)}: {worst:.3e}"
        assert np.abs(got - default).max() <= 1e-5 * np.abs(default).max()
    y = torch.empty((rows, n), dtype=torch.float32, device=cuda)
    with pytest.raises(_lib.VxError) as info:  # 16 waves of 4 row groups: no such kernel
        _lib.check(_lib.lib().vx_q8_linear_engine(x_dev.data_ptr(), packed.data_ptr(),
                                                  y.data_ptr(), rows, k, n, 4, 16, 1, 1, handle))
    assert info.value.status == _lib.VX_UNSUPPORTED


@pytest.mark.parametrize("rows", [33, 44, 64, 100, 128])
def test_products_beyond_32_rows(vx, oracle, cuda, stream, rows):
    """33..128 rows stay exact (the reference's chunks of 32, gemm.cpp:272)."""
    k, n = 1024, 2560
    rng = synth.Rng(99, rows)
    blocks = reference_weights(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x = reference_activations(rng, rows, k)
    before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
    scratch = vx.Scratch(128, n)
    for accumulate in (False, True):
        y = run_product(vx, to_device(x, cuda), packed, n,
                        before if accumulate else None, None, scratch, cuda)
        assert oracle.q8_check(y, x, blocks, before if accumulate else None) <= LIMIT


@pytest.mark.parametrize("rows,k,n", [(100, 1024, 16400), (128, 2048, 16384)])
def test_wide_products_beyond_64_rows(vx, oracle, cuda, stream, rows, k, n):
    """More than 64 rows over wide outputs take blocks of up to 64 rows,
    each staged per wave, with the exact per-block arithmetic (ragged rows
    and columns, a tile count that is not a multiple of 8, and
    accumulation)."""
    rng = synth.Rng(77, rows + n)
    blocks = reference_weights(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x = reference_activations(rng, rows, k)
    before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
    scratch = vx.Scratch(128, n)
    cols = np.arange(0, n, 5)
    for accumulate in (False, True):
        y = run_product(vx, to_device(x, cuda), packed, n,
                        before if accumulate else None, None, scratch, cuda)
        worst = oracle.q8_check(np.ascontiguousarray(y[:, cols]), x,
                                np.ascontiguousarray(blocks[cols]),
                                np.ascontiguousarray(before[:, cols]) if accumulate else None)
        assert worst <= LIMIT, f"accumulate {accumulate}: worst {worst:.3e}"


@pytest.mark.parametrize("rows,k,n", [(22, 1024, 4096),
                                      # the prefill kernel, ragged rows and columns
                                      (600, 1024, 6160)])
def test_bf16_output_is_rounded_float_output(vx, cuda, stream, rows, k, n):
    rng = synth.Rng(0, 3)
    blocks = synth.q8_blocks(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x_dev = to_device(synth.activations(rng, rows, k), cuda)
    scratch = vx.Scratch(min(rows, 128), n)
    y32 = vx.q8_linear(x_dev, packed, n, scratch=scratch)
    y16 = vx.q8_linear_bf16(x_dev, packed, n, scratch=scratch)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_host(y16), synth.bf16_bits(y32.cpu().numpy()))


@pytest.mark.parametrize("k,n", [(1024, 3072), (1024, 8192), (2048, 2048),
                                 (2048, 16384), (1024, 4096)])
@pytest.mark.parametrize("rows", [1, 2, 22, 44, 128])
def test_sweep_shapes_baseline_law(vx, oracle, cuda, stream, k, n, rows):
    """The benchmark sweep's shapes with its weight law (30 % of the float16
    scales subnormal): the error bound holds for every row count."""
    rng = synth.Rng(0, 1000 * rows + n + k)
    blocks = synth.q8_blocks(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x = synth.activations(rng, rows, k)
    scratch = vx.Scratch(128, n)
    y = run_product(vx, to_device(x, cuda), packed, n, None, None, scratch, cuda)
    # Every 7th output column (all lanes and row groups are visited) keeps
    # the double-precision check within seconds.
    cols = np.arange(0, n, 7)
    assert oracle.q8_check(np.ascontiguousarray(y[:, cols]), x,
                           np.ascontiguousarray(blocks[cols])) <= LIMIT


@pytest.mark.parametrize("k,n", [(1024, 8192), (2048, 16384), (1024, 16400)])
@pytest.mark.parametrize("rows", [17, 22, 32])
def test_wide_plans_accumulate(vx, oracle, cuda, stream, k, n, rows):
    """17-32 rows over 512 or more row groups take the eight-wave plans (one
    or two row groups per workgroup, two pairs in flight with two; four
    row groups past 1024, here with a partial last tile): y += x W^T and
    the plain store both within the bound, checked on every 7th column
    (all lanes and row groups are visited)."""
    rng = synth.Rng(31, 100 * rows + n + k)
    blocks = reference_weights(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    plan = vx.q8_plan(rows, k, n)
    assert plan["waves"] == 8, plan
    x = reference_activations(rng, rows, k)
    x_dev = to_device(x, cuda)
    before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
    cols = np.arange(0, n, 7)
    for accumulate in (False, True):
        y = run_product(vx, x_dev, packed, n, before if accumulate else None, None, None, cuda)
        worst = oracle.q8_check(np.ascontiguousarray(y[:, cols]), x,
                                np.ascontiguousarray(blocks[cols]),
                                np.ascontiguousarray(before[:, cols]) if accumulate else None)
        assert worst <= LIMIT, (rows, k, n, accumulate, worst)


def expanded_check(y, x, blocks, oracle, before=None):
    """Error of y against the reference's expansion (gemm.cpp:305-312):
    x . bf16(scale q) in double, relative to sum |x w|."""
    m, k = x.shape
    n = y.shape[1]
    w = synth.bf16_values(oracle.q8_dequant_bf16(blocks, n, k)).astype(np.float64)
    xf = synth.bf16_values(x).astype(np.float64)
    exact = xf @ w.T
    if before is not None:
        exact += before
    magnitude = np.abs(xf) @ np.abs(w).T
    return float(np.max(np.abs(y - exact) / np.maximum(magnitude, 1e-30)))


@pytest.mark.parametrize("rows,k,n", [(129, 2048, 2048), (256, 2048, 6144),
                                      (300, 1024, 2560), (512, 2048, 2048),
                                      (1024, 2048, 1040),
                                      # 128-row tiles, ragged rows and columns
                                      (700, 1024, 4112),
                                      # columns not a multiple of 4 (the split
                                      # reduction's scalar path)
                                      (200, 512, 1042),
                                      # the prefill kernel's ragged rows and
                                      # columns (256-row, 128/256-column tiles)
                                      (700, 1024, 6160)])
def test_prefill_expansion(vx, oracle, cuda, stream, rows, k, n):
    """More than 128 rows: W as bf16(scale * q), float32 sums; the
    reference allows 1e-4 there (products_test.cpp:301-309)."""
    rng = synth.Rng(4, rows + n)
    blocks = synth.q8_blocks(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x = synth.activations(rng, rows, k)
    before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
    # Without a scratch one pass over k; with one, small grids split k over
    # workgroups and add the splits in order in a second launch.
    scratch = vx.Scratch(128, max(n, 4096))
    results = []
    for use_scratch in (None, scratch):
        for accumulate in (False, True):
            y = run_product(vx, to_device(x, cuda), packed, n,
                            before if accumulate else None, None, use_scratch, cuda)
            worst = expanded_check(y, x, blocks, oracle, before if accumulate else None)
            assert worst <= 1e-4, f"scratch {use_scratch is not None}: worst {worst:.3e}"
            results.append(y)
    # A split product repeats bit for bit.
    again = run_product(vx, to_device(x, cuda), packed, n, None, None, scratch, cuda)
    assert np.array_equal(again, results[2])


@pytest.mark.parametrize("n", [2048, 6144, 16384])
@pytest.mark.parametrize("rows", [129, 256, 512, 1024])
def test_prefill_benched_shapes(vx, oracle, cuda, stream, rows, n):
    """Every prefill shape the benchmark times (K = 2048), called as it calls
    them (with a product scratch), against the expanded arithmetic in double
    at the reference's 1e-4 (products_test.cpp:279-310). Every 7th output
    column is checked (7 is prime to the 16-column groups and 128-column
    tiles, so every lane and tile position is visited)."""
    k = 2048
    rng = synth.Rng(7, n * 10 + rows)
    blocks = synth.q8_blocks(rng, n, k)
    packed = vx.q8_pack(to_device(blocks, cuda), n, k)
    x = synth.activations(rng, rows, k)
    scratch = vx.Scratch(128, 16384)
    y = run_product(vx, to_device(x, cuda), packed, n, None, None, scratch, cuda)
    cols = np.arange(0, n, 7)
    worst = expanded_check(np.ascontiguousarray(y[:, cols]), x,
                           np.ascontiguousarray(blocks[cols]), oracle)
    print(f"prefill {rows}x{k}x{n}: worst {worst:.2e}", flush=True)
    assert worst <= 1e-4


def test_stream_read_reads_every_byte(vx, cuda, stream):
    """The read-ceiling kernel loads every 16-byte chunk: the XOR of the
    buffer's words reaches the sink only when it equals `never`."""
    words = np.arange(1, 4096 * 4 + 1, dtype=np.uint32) * np.uint32(2654435761)
    data = torch.from_numpy(words.view(np.int32)).to(cuda)
    chunk_xor = np.bitwise_xor.reduce(words.reshape(-1, 4), axis=1)
    sink = torch.zeros(1, dtype=torch.int32, device=cuda)
    # `never` equal to one chunk's XOR: exactly that chunk writes it.
    target = int(chunk_xor[1234])
    vx.stream_read(data, sink, never=target)
    torch.cuda.synchronize()
    assert int(sink.cpu().numpy().view(np.uint32)[0]) == target
    sink.zero_()
    missing = int(np.uint32(0xFFFFFFFF))
    assert missing not in set(chunk_xor.tolist())
    vx.stream_read(data, sink, never=missing)
    torch.cuda.synchronize()
    assert int(sink.cpu().numpy()[0]) == 0
