"""bfloat16-weight panels and products on the GPU against the CPU oracle.

Mirrors the reference's bf16 checks in tests/products_test.cpp: the weights
are the bf16 expansion of random GGML Q8_0 blocks (the reference's bf16
tiles, :155-190) or bf16 ~ N(0, 1), the activations bf16 ~ N(0, 2), every
row count up to 32 and past it, with and without accumulation; each output
is compared with a double-precision sum, its error relative to sum |x w|
at most 1e-5 (:117-145, 234-237, 300-308). The panel layout's round trip
is bit-exact, including NaN, infinite and subnormal bit patterns.
"""
import numpy as np
import pytest
import torch

from voxcpm_amd import synth
from test_products_gpu import (ALL_ROWS, LIMIT, SHAPES, bf16_host, reference_activations,
                               reference_weights, to_device)

pytestmark = pytest.mark.gpu


def bf16_weights(oracle, rng: synth.Rng, n: int, k: int, dequantized: bool) -> np.ndarray:
    """bf16 bits [n][k]: bf16(scale q) of random Q8_0 blocks, or N(0, 1)."""
    if dequantized:
        return oracle.q8_dequant_bf16(reference_weights(rng, n, k), n, k)
    return synth.bf16_bits(rng.normal(n * k).astype(np.float32)).reshape(n, k)


def panel_bytes(rows: np.ndarray) -> np.ndarray:
    """The panel layout restated on the host: unit (g, p) = 2048 bytes, half
    h, lane L = 16 j + r: w[16 g + r][64 p + 32 h + 8 j + 0..7], zero past
    the matrix."""
    n, k = rows.shape
    groups, pairs = (n + 15) // 16, (k + 63) // 64
    padded = np.zeros((groups * 16, pairs * 64), dtype=np.uint16)
    padded[:n, :k] = rows
    # [g][r][p][h][j][8] -> [g][p][h][j][r][8]
    blocks = padded.reshape(groups, 16, pairs, 2, 4, 8).transpose(0, 2, 3, 4, 1, 5)
    return np.ascontiguousarray(blocks).reshape(-1).view(np.uint8)


@pytest.mark.parametrize("k,n", [(32, 16), (64, 17), (96, 40), (1024, 72), (160, 2)])
def test_bf16_pack_round_trip_and_layout(vx, cuda, stream, k, n):
    rng = synth.Rng(99, 13 * k + n)
    rows = (rng.bits(n * k) & np.uint64(0xFFFF)).astype(np.uint16).reshape(n, k)
    # NaN, infinities, subnormals and signed zeros among the bit patterns
    special = np.array([0x7FC1, 0xFF80, 0x7F80, 0x0001, 0x8001, 0x0000, 0x8000, 0x007F],
                       dtype=np.uint16)
    rows.reshape(-1)[: special.size] = special
    packed = vx.bf16_pack(to_device(rows, cuda))
    assert packed.numel() == ((n + 15) // 16) * ((k + 63) // 64) * 2048
    back = vx.bf16_unpack(packed, n, k)
    torch.cuda.synchronize()
    assert np.array_equal(bf16_host(back), rows), "pack/unpack round trip"
    assert np.array_equal(packed.cpu().numpy(), panel_bytes(rows)), "panel layout"


def run(vx, x_dev, packed, n, before, scratch, cuda):
    y = torch.from_numpy(before.copy()).to(cuda) if before is not None else None
    out = vx.bf16_linear(x_dev, packed, n, y=y, accumulate=before is not None, scratch=scratch)
    torch.cuda.synchronize()
    return out.cpu().numpy()


@pytest.mark.parametrize("k,n,rows_list", SHAPES)
def test_bf16_products_against_double(vx, oracle, cuda, stream, k, n, rows_list):
    rng = synth.Rng(4321, 10 * k + n)
    w = bf16_weights(oracle, rng, n, k, dequantized=True)
    packed = vx.bf16_pack(to_device(w, cuda))
    scratch = vx.Scratch(32, n)
    for rows in rows_list:
        x = reference_activations(rng, rows, k)
        x_dev = to_device(x, cuda)
        before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
        y = run(vx, x_dev, packed, n, None, scratch, cuda)
        error = oracle.bf16_check(y, x, w)
        assert error <= LIMIT, f"rows {rows}: {error:.3e}"
        y2 = run(vx, x_dev, packed, n, before, scratch, cuda)
        error = oracle.bf16_check(y2, x, w, before)
        assert error <= LIMIT, f"rows {rows} (accumulate): {error:.3e}"
        # The same bits on a second run.
        assert np.array_equal(y, run(vx, x_dev, packed, n, None, scratch, cuda))


@pytest.mark.parametrize("k,n,rows_list", [
    (1024, 2560, [40, 64, 100, 128]),   # the engine, one and two row blocks
    (2048, 2048, [129, 256]),           # past 128 rows (hipBLASLt's in the reference)
    (96, 40, [65, 130]),                # odd pair count, rows not a multiple of 16
    (2048, 16384, [44, 128]),           # four row groups per workgroup; two row blocks
])
def test_bf16_products_many_rows(vx, oracle, cuda, stream, k, n, rows_list):
    rng = synth.Rng(77, k + n)
    w = bf16_weights(oracle, rng, n, k, dequantized=False)
    packed = vx.bf16_pack(to_device(w, cuda))
    scratch = vx.Scratch(128, n)
    for rows in rows_list:
        x = reference_activations(rng, rows, k)
        x_dev = to_device(x, cuda)
        before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
        for s in (None, scratch):
            y = run(vx, x_dev, packed, n, None, s, cuda)
            error = oracle.bf16_check(y, x, w)
            assert error <= LIMIT, f"rows {rows}: {error:.3e}"
        y2 = run(vx, x_dev, packed, n, before, scratch, cuda)
        error = oracle.bf16_check(y2, x, w, before)
        assert error <= LIMIT, f"rows {rows} (accumulate): {error:.3e}"


@pytest.mark.parametrize("k,n,rows_list", [
    (1024, 2560, ALL_ROWS),
    (2048, 1024, [1, 5, 22]),
    (72, 40, [1, 7, 16, 17, 32]),   # k a multiple of 8 only: a short last block
    (8, 3, [2]),
    (4096, 33, [1, 22]),
])
def test_bf16_rows_products_against_double(vx, oracle, cuda, stream, k, n, rows_list):
    """Row-major bf16 weights as they come (the reference's SkinnyGemm)."""
    rng = synth.Rng(55, k * 3 + n)
    w = bf16_weights(oracle, rng, n, k, dequantized=False)
    w_dev = to_device(w, cuda)
    for rows in rows_list:
        x = reference_activations(rng, rows, k)
        x_dev = to_device(x, cuda)
        before = rng.normal(rows * n).astype(np.float32).reshape(rows, n)
        y = vx.bf16_linear_rows(x_dev, w_dev)
        torch.cuda.synchronize()
        error = oracle.bf16_check(y.cpu().numpy(), x, w)
        assert error <= LIMIT, f"rows {rows}: {error:.3e}"
        y2 = torch.from_numpy(before.copy()).to(cuda)
        vx.bf16_linear_rows(x_dev, w_dev, y=y2, accumulate=True)
        torch.cuda.synchronize()
        error = oracle.bf16_check(y2.cpu().numpy(), x, w, before)
        assert error <= LIMIT, f"rows {rows} (accumulate): {error:.3e}"


def test_bf16_rows_limits(vx, cuda, stream):
    """More than 32 rows is unsupported (the reference hands those to
    hipBLASLt), as are k not a multiple of 8; nothing is launched."""
    from voxcpm_amd import _lib
    w = torch.zeros((16, 64), dtype=torch.bfloat16, device=cuda)
    with pytest.raises(_lib.VxError) as info:
        vx.bf16_linear_rows(torch.zeros((33, 64), dtype=torch.bfloat16, device=cuda), w)
    assert info.value.status == _lib.VX_UNSUPPORTED
    with pytest.raises(_lib.VxError) as info:
        vx.bf16_linear_rows(torch.zeros((2, 60), dtype=torch.bfloat16, device=cuda),
                            torch.zeros((16, 60), dtype=torch.bfloat16, device=cuda))
    assert info.value.status == _lib.VX_BAD_ARG
