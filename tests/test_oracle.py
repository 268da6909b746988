"""Pins the CPU oracle (oracle/oracle.c) against what fixes it independently:
library conversions (numpy float16, torch bfloat16), torch.linspace (which
the reference's Linspace mirrors, generator.cpp:21-22), closed forms and
invariants, brute force in float64 on small inputs, and a float64 torch
formulation of the whole DiT. Each check is chosen so that a plausible slip
(a dropped term, a swapped operand, a wrong index, a wrong rounding) fails.
"""
import ctypes
import math

import numpy as np
import pytest
import torch

from voxcpm_amd import synth


def f32(x):
    return np.ascontiguousarray(x, dtype=np.float32)


# ---- conversions ------------------------------------------------------------

def test_bf16_rounding_matches_torch(oracle):
    rng = synth.Rng(1, 1)
    bits = rng.bits(200000).astype(np.uint32)
    values = bits.view(np.float32)
    values = values[np.isfinite(values)]
    # ties: the low 16 bits exactly 0x8000, odd and even upper halves
    ties = (np.arange(0, 2000, dtype=np.uint32) << 16 | 0x8000).view(np.float32)
    values = f32(np.concatenate([values, ties, [0.0, -0.0, 1e-45, 3.4e38, -3.4e38]]))
    out = np.zeros(values.size, dtype=np.uint16)
    oracle.lib().vo_bf16_round_array(oracle.ptr(values), oracle.ptr(out), values.size)
    expected = torch.from_numpy(values).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(out, expected.view(np.uint16))
    # NaNs stay quiet NaNs with the payload's upper half.
    nan = np.array([0x7F800001, 0xFF812345, 0x7FC00000], dtype=np.uint32).view(np.float32)
    for value, bits_in in zip(nan, [0x7F800001, 0xFF812345, 0x7FC00000]):
        assert oracle.lib().vo_bf16_bits(float(value)) == ((bits_in >> 16) | 0x40)


def test_half_decode_exhaustive(oracle):
    bits = np.arange(65536, dtype=np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib().vo_half_value(int(b)) for b in bits], dtype=np.float32)
    finite = np.isfinite(expected)
    assert np.array_equal(got[finite].view(np.uint32), expected[finite].view(np.uint32))
    assert np.array_equal(np.isnan(got), np.isnan(expected))
    assert np.array_equal(np.isinf(got), np.isinf(expected))


def test_half_encode_matches_numpy(oracle):
    rng = synth.Rng(2, 2)
    values = f32(np.concatenate([rng.normal(20000, 1e-3), rng.normal(20000, 1e-6),
                                 rng.normal(2000, 1e4), [65519.0, 65520.0, 6e-8, 3e-8]]))
    got = np.array([oracle.lib().vo_half_bits(float(v)) for v in values], dtype=np.uint16)
    assert np.array_equal(got, values.astype(np.float16).view(np.uint16))


# ---- Q8_0 -----------------------------------------------------------------------

def test_q8_dequant_closed_form(oracle):
    rng = synth.Rng(3, 3)
    n, k = 48, 128
    blocks = synth.q8_blocks(rng, n, k)
    blocks.reshape(-1, 34)[::5, 2] = 0x80  # q = -128
    got = oracle.q8_dequant_bf16(blocks, n, k)
    scale = blocks[:, :, :2].copy().view(np.uint16).view(np.float16).astype(np.float32)
    q = blocks[:, :, 2:].view(np.int8).astype(np.float32)
    exact = (scale * q).reshape(n, k)  # exact in float32 (19 significant bits)
    expected = torch.from_numpy(exact).to(torch.bfloat16).view(torch.int16).numpy()
    assert np.array_equal(got, expected.view(np.uint16))
    values = oracle.q8_values(blocks, n, k)
    assert np.array_equal(values, exact.astype(np.float64))


def test_q8_linear_exact_on_integers(oracle):
    """Unit scales and small integer activations: every float32 sum is exact,
    so the product equals the integer matrix product bit for bit."""
    rng = synth.Rng(4, 4)
    m, k, n = 5, 256, 40
    blocks = synth.q8_blocks(rng, n, k)
    flat = blocks.reshape(-1, 34)
    flat[:, 0] = 0x00
    flat[:, 1] = 0x3C  # 1.0
    xi = ((rng.bits(m * k) % np.uint64(9)).astype(np.int64) - 4).reshape(m, k)
    x = synth.bf16_bits(xi.astype(np.float32))
    y = oracle.q8_linear(x, blocks, n, threads=3)
    q = blocks[:, :, 2:].view(np.int8).astype(np.int64).reshape(n, k)
    assert np.array_equal(y, (xi @ q.T).astype(np.float32))


def test_q8_linear_block_scales_and_accumulate(oracle):
    """Against a float64 product of the dequantized values (independent of the
    oracle's loops) and the accumulate path: y = before + x W^T."""
    rng = synth.Rng(5, 5)
    m, k, n = 7, 320, 33
    blocks = synth.q8_blocks(rng, n, k)
    x = synth.activations(rng, m, k)
    w = oracle.q8_values(blocks, n, k)
    xf = synth.bf16_values(x).astype(np.float64)
    exact = xf @ w.T
    magnitude = np.abs(xf) @ np.abs(w).T
    y = oracle.q8_linear(x, blocks, n, threads=4)
    assert np.max(np.abs(y - exact) / magnitude) < 2e-6
    before = f32(rng.normal(m * n).reshape(m, n))
    y2 = oracle.q8_linear(x, blocks, n, before=before, threads=1)
    assert np.max(np.abs(y2 - (exact + before)) / (magnitude + np.abs(before))) < 2e-6
    # The checker agrees, and catches a planted error of 1e-4 |x w|.
    assert oracle.q8_check(y, x, blocks) < 2e-6
    bad = y.copy()
    bad[3, 7] += 1e-4 * magnitude[3, 7]
    assert oracle.q8_check(bad, x, blocks) > 5e-5
    # Thread count does not change a bit.
    assert np.array_equal(y, oracle.q8_linear(x, blocks, n, threads=1))


def test_q8_linear_scales_after_block_sums(oracle):
    """The scale multiplies each block's float32 sum (fmaf), not each value:
    a block whose exact sum is zero contributes exactly zero even with a
    scale whose products with q are inexact in bf16."""
    k, n = 64, 1
    blocks = np.zeros((n, k // 32, 34), dtype=np.uint8)
    blocks[0, :, 0:2] = np.frombuffer(np.float16(0.0123).tobytes(), np.uint8)
    q = np.zeros(32, dtype=np.int8)
    q[0], q[1] = 77, -77
    blocks[0, 0, 2:] = q.view(np.uint8)
    blocks[0, 1, 2:] = q.view(np.uint8)
    x = synth.bf16_bits(f32(np.ones((1, k))))
    y = oracle.q8_linear(x, blocks, n)
    assert y[0, 0] == 0.0


def test_bf16_linear_exact_on_integers(oracle):
    """Small integer activations and weights in bf16: every float32 sum is
    exact, so the product equals the integer matrix product bit for bit."""
    rng = synth.Rng(6, 6)
    m, k, n = 4, 96, 21
    xi = ((rng.bits(m * k) % np.uint64(9)).astype(np.int64) - 4).reshape(m, k)
    wi = ((rng.bits(n * k) % np.uint64(15)).astype(np.int64) - 7).reshape(n, k)
    x = synth.bf16_bits(xi.astype(np.float32))
    w = synth.bf16_bits(wi.astype(np.float32))
    assert np.array_equal(oracle.bf16_linear(x, w), (xi @ wi.T).astype(np.float32))


@pytest.mark.parametrize("k", [64, 40])
def test_bf16_linear_against_float64(oracle, k):
    """Against a float64 product (independent of the oracle's loops), a k
    with a short last 16-column chunk, and the accumulate path; the checker
    agrees and catches a planted error of 1e-4 |x w|."""
    rng = synth.Rng(7, k)
    m, n = 6, 19
    x = synth.activations(rng, m, k)
    w = synth.activations(rng, n, k)
    xf = synth.bf16_values(x).astype(np.float64)
    wf = synth.bf16_values(w).astype(np.float64)
    exact = xf @ wf.T
    magnitude = np.abs(xf) @ np.abs(wf).T
    y = oracle.bf16_linear(x, w)
    assert np.max(np.abs(y - exact) / magnitude) < 2e-6
    before = f32(rng.normal(m * n).reshape(m, n))
    y2 = oracle.bf16_linear(x, w, before=before)
    assert np.max(np.abs(y2 - (exact + before)) / (magnitude + np.abs(before))) < 2e-6
    assert oracle.bf16_check(y, x, w) < 2e-6
    assert oracle.bf16_check(y2, x, w, before) < 2e-6
    bad = y.copy()
    bad[2, 5] += 1e-4 * magnitude[2, 5]
    assert oracle.bf16_check(bad, x, w) > 5e-5
    # A transposed weight (a plausible layout slip) fails the checker.
    if k == 64:
        assert oracle.bf16_check(oracle.bf16_linear(x, np.ascontiguousarray(w[::-1])), x, w) > 1e-2


# ---- generator kernels -------------------------------------------------------

def test_rms_norm(oracle):
    rng = synth.Rng(6, 6)
    rows, width, eps = 3, 1024, 1e-5
    x = f32(rng.normal(rows * width, 3.0).reshape(rows, width))
    x[2] = 0.5  # constant row: closed form gamma * c / sqrt(c^2 + eps)
    gamma = synth.bf16_vector(rng, width, 1.0, 0.02)
    out = np.zeros((rows, width), dtype=np.uint16)
    out32 = np.zeros((rows, width), dtype=np.float32)
    oracle.lib().vo_rms_norm(oracle.ptr(x), oracle.ptr(gamma), oracle.ptr(out),
                             oracle.ptr(out32), rows, width, eps)
    g = synth.bf16_values(gamma).astype(np.float64)
    xd = x.astype(np.float64)
    expected = xd / np.sqrt((xd ** 2).mean(axis=1, keepdims=True) + eps) * g
    assert np.max(np.abs(out32 - expected)) < 1e-5 * np.abs(expected).max()
    assert np.allclose(out32[2], g * 0.5 / math.sqrt(0.25 + eps), rtol=1e-6)
    assert np.array_equal(out, synth.bf16_bits(out32))


def test_rope_table_and_rotation(oracle):
    dim, positions = 128, 11
    factors = np.array(synth.VOXCPM2_SHORT_FACTORS)
    table = oracle.rope_table(10000.0, dim, factors, 1.0, positions)
    half = dim // 2
    i = np.arange(half)
    angle = np.arange(positions)[:, None] / factors[None, :] * 10000.0 ** (-2.0 * i / dim)
    assert np.max(np.abs(table[:, :half] - np.cos(angle))) < 2e-5
    assert np.max(np.abs(table[:, half:] - np.sin(angle))) < 2e-5
    assert np.array_equal(table[0, :half], np.ones(half, np.float32))
    assert np.array_equal(table[0, half:], np.zeros(half, np.float32))
    # QkvRope: rotation of pairs (i, i + half); position 0 is the identity,
    # norms of the pairs are kept, and <R(p) q, R(p') k> depends on p - p'.
    rng = synth.Rng(7, 7)
    heads, kv_heads, rows = 2, 1, 4
    width = (heads + 2 * kv_heads) * dim
    base = f32(rng.normal(width))
    qkv = f32(np.tile(base, (rows, 1)))
    positions_arr = np.array([0, 3, 5, 8], dtype=np.int32)
    cache_rows = np.array([0, 1, 2, 3], dtype=np.int32)
    q = np.zeros((rows, heads, dim), np.float32)
    kc = np.zeros((kv_heads, rows, dim), np.float32)
    vc = np.zeros((kv_heads, rows, dim), np.float32)
    oracle.lib().vo_qkv_rope(oracle.ptr(qkv), oracle.ptr(table), oracle.ptr(positions_arr),
                             oracle.ptr(cache_rows), oracle.ptr(q), oracle.ptr(kc),
                             oracle.ptr(vc), rows, heads, kv_heads, dim, rows)
    assert np.array_equal(q[0].ravel(), base[:heads * dim])
    assert np.array_equal(vc[0, 2], base[(heads + kv_heads) * dim:])
    for r in range(rows):
        a, b = q[r, 1, :half].astype(np.float64), q[r, 1, half:].astype(np.float64)
        a0, b0 = base[dim:dim + half].astype(np.float64), base[dim + half:2 * dim].astype(np.float64)
        assert np.allclose(a * a + b * b, a0 * a0 + b0 * b0, rtol=1e-5)
    # q at position 8 against k at 5 equals q at 3 against k at 0.
    d1 = float(np.dot(q[3, 0].astype(np.float64), kc[0, 2].astype(np.float64)))
    d2 = float(np.dot(q[1, 0].astype(np.float64), kc[0, 0].astype(np.float64)))
    assert abs(d1 - d2) < 1e-4 * max(1.0, abs(d1))


@pytest.mark.parametrize("head_dim,heads,kv_heads", [(64, 4, 4), (128, 4, 2), (32, 3, 1)])
def test_attention_against_torch(oracle, head_dim, heads, kv_heads):
    rng = synth.Rng(8, head_dim)
    length, rows = 11, 22
    q = f32(rng.normal(rows * heads * head_dim).reshape(rows, heads, head_dim))
    kc = f32(rng.normal(kv_heads * rows * head_dim).reshape(kv_heads, rows, head_dim))
    vc = f32(rng.normal(kv_heads * rows * head_dim).reshape(kv_heads, rows, head_dim))
    out = np.zeros((rows, heads, head_dim), np.uint16)
    oracle.lib().vo_attention(oracle.ptr(q), oracle.ptr(kc), oracle.ptr(vc), oracle.ptr(out),
                              rows, length, length, 0, 0, heads, kv_heads, head_dim, rows)
    got = synth.bf16_values(out).astype(np.float64)
    group = heads // kv_heads
    for s in range(2):
        rs = slice(s * length, (s + 1) * length)
        qt = torch.from_numpy(q[rs].astype(np.float64)).permute(1, 0, 2)
        kt = torch.from_numpy(kc[:, rs].astype(np.float64)).repeat_interleave(group, 0)
        vt = torch.from_numpy(vc[:, rs].astype(np.float64)).repeat_interleave(group, 0)
        ref = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt).permute(1, 0, 2).numpy()
        assert np.max(np.abs(got[rs] - ref)) < 1e-2 * np.abs(ref).max()
    # causal with one key: the output is that key's value
    out1 = np.zeros((1, heads, head_dim), np.uint16)
    oracle.lib().vo_attention(oracle.ptr(q), oracle.ptr(kc), oracle.ptr(vc), oracle.ptr(out1),
                              1, 1, 1, 0, 1, heads, kv_heads, head_dim, rows)
    for h in range(heads):
        assert np.array_equal(out1[0, h], synth.bf16_bits(vc[h // group, 0]))


def test_swiglu_bias_to_bf16(oracle):
    rng = synth.Rng(9, 9)
    rows, width = 3, 256
    gu = f32(rng.normal(rows * 2 * width, 3.0).reshape(rows, 2 * width))
    out = np.zeros((rows, width), np.uint16)
    oracle.lib().vo_swiglu(oracle.ptr(gu), oracle.ptr(out), rows, width)
    g = torch.from_numpy(gu[:, :width].astype(np.float64))
    u = torch.from_numpy(gu[:, width:].astype(np.float64))
    ref = (torch.nn.functional.silu(g) * u).numpy()
    got = synth.bf16_values(out)
    assert np.all(np.abs(got - ref) <= np.abs(ref) * 2 ** -8 + 1e-30)
    bias = synth.bf16_vector(rng, width, 0.0, 0.5)
    data = f32(rng.normal(rows * width).reshape(rows, width))
    before = data.copy()
    oracle.lib().vo_add_bias(oracle.ptr(data), oracle.ptr(bias), rows, width)
    assert np.array_equal(data, before + synth.bf16_values(bias)[None, :])
    silu = np.zeros(rows * width, np.uint16)
    oracle.lib().vo_to_bf16(oracle.ptr(before), oracle.ptr(silu), rows * width, 1)
    ref = torch.nn.functional.silu(torch.from_numpy(before.astype(np.float64))).numpy().ravel()
    assert np.all(np.abs(synth.bf16_values(silu) - ref) <= np.abs(ref) * 2 ** -8 + 1e-30)


def test_assemble_and_gather(oracle):
    patch, width = 4, 8
    mu = f32(np.arange(2 * width) + 100)
    time = f32(np.arange(width) + 200)
    cond = f32(np.arange(patch * width).reshape(patch, width) + 300)
    x = f32(np.arange(patch * width).reshape(patch, width) + 400)
    out = np.zeros((2, 11, width), np.float32)
    oracle.lib().vo_assemble_dit(oracle.ptr(mu), oracle.ptr(time), oracle.ptr(cond),
                                 oracle.ptr(x), oracle.ptr(out), patch, width)
    assert np.array_equal(out[0, 0:2].ravel(), mu)
    assert np.array_equal(out[1, 0:2], np.zeros((2, width)))
    for s in range(2):
        assert np.array_equal(out[s, 2], time)
        assert np.array_equal(out[s, 3:7], cond)
        assert np.array_equal(out[s, 7:11], x)
    idx = np.array([7, 8, 9, 10, 18, 19, 20, 21], dtype=np.int32)
    gathered = np.zeros((8, width), np.float32)
    oracle.lib().vo_gather_rows(oracle.ptr(out.reshape(22, width)), oracle.ptr(idx),
                                oracle.ptr(gathered), 8, width)
    assert np.array_equal(gathered, np.concatenate([x, x]))


def test_guided_euler_closed_forms(oracle):
    rng = synth.Rng(10, 10)
    count = 256
    c = f32(rng.normal(count))
    u = f32(rng.normal(count))
    v = f32(np.concatenate([c, u]))
    x0 = f32(rng.normal(count))
    # plain CFG (s = 1): x -= dt (u + cfg (c - u))
    x = x0.copy()
    oracle.lib().vo_guided_euler(oracle.ptr(v), oracle.ptr(x), count, 2.0, 0.1, 0)
    ref = x0.astype(np.float64) - 0.1 * (u + 2.0 * (c.astype(np.float64) - u))
    assert np.allclose(x, ref, atol=1e-6)
    # cfg = 1, s = 1: x -= dt c
    x = x0.copy()
    oracle.lib().vo_guided_euler(oracle.ptr(v), oracle.ptr(x), count, 1.0, 0.25, 0)
    assert np.allclose(x, x0 - 0.25 * c, atol=1e-6)
    # CFG-Zero*: s = <c,u>/(|u|^2 + 1e-8); with c = u, v = u for any cfg
    x = x0.copy()
    same = f32(np.concatenate([u, u]))
    oracle.lib().vo_guided_euler(oracle.ptr(same), oracle.ptr(x), count, 2.0, 0.5, 1)
    assert np.allclose(x, x0 - 0.5 * u, atol=1e-5)
    x = x0.copy()
    oracle.lib().vo_guided_euler(oracle.ptr(v), oracle.ptr(x), count, 2.0, 0.1, 1)
    s = np.dot(c.astype(np.float64), u) / (np.dot(u.astype(np.float64), u) + 1e-8)
    ref = x0 - 0.1 * (u * s + 2.0 * (c - u * s))
    assert np.allclose(x, ref, atol=1e-5)


# ---- sampler ---------------------------------------------------------------------

@pytest.mark.parametrize("steps", [1, 2, 3, 10, 11, 25, 101])
def test_linspace_matches_torch(oracle, steps):
    out = np.zeros(steps, np.float32)
    oracle.lib().vo_linspace(1.0, 0.0, steps, oracle.ptr(out))
    expected = torch.linspace(1.0, 0.0, steps, dtype=torch.float32).numpy()
    assert np.array_equal(out, expected)


def test_euler_schedule(oracle):
    # Uniform (sway 0), no skip: t = 1 - i/10 from torch.linspace, dt = 0.1.
    t, dt, ev = oracle.euler_schedule(10, 0.0, False)
    lin = torch.linspace(1.0, 0.0, 11, dtype=torch.float32).numpy()
    assert np.array_equal(t[0:1], lin[0:1])
    assert np.allclose(t, lin[:10], atol=1e-6)
    assert np.allclose(dt, 0.1, atol=1e-6)
    assert ev.tolist() == [1] * 10
    # The chained t stays within float32 rounding of the span and the dt
    # sum to 1 (the end point 0).
    assert abs(float(np.sum(dt.astype(np.float64))) - 1.0) < 1e-6
    # Sway 1 and CFG-Zero*'s skip: t = s + (cos(pi s / 2) - 1 + s); the
    # first max(1, int(0.04 * 11)) = 1 step is not evaluated.
    t, dt, ev = oracle.euler_schedule(10, 1.0, True)
    span = lin.astype(np.float64)
    warped = span + (np.cos(np.pi / 2 * span) - 1 + span)
    assert np.allclose(t, warped[:10], atol=2e-6)
    assert np.allclose(dt, warped[:10] - warped[1:], atol=2e-6)
    assert ev.tolist() == [0] + [1] * 9
    # t of the reference's 10-step schedule (restated from generator.cpp)
    table = [1.0, 0.9564344, 0.9090170, 0.8539906, 0.7877852, 0.7071068,
             0.6090170, 0.4910066, 0.3510565, 0.1876884]
    assert np.allclose(t, table, atol=1e-6)
    # 25 steps skip int(0.04 * 26) = 1; 50 steps skip int(2.04) = 2
    assert oracle.euler_schedule(50, 1.0, True)[2][:3].tolist() == [0, 0, 1]


def test_sinusoid(oracle):
    for t, width in [(0.0, 256), (0.63, 1024), (1.0, 256), (0.1876884, 1024)]:
        out = np.zeros(width, np.float32)
        oracle.lib().vo_sinusoid(t, width, oracle.ptr(out))
        half = width // 2
        freq = np.exp(-np.arange(half) * math.log(10000.0) / (half - 1))
        angle = 1000.0 * t * freq
        assert np.max(np.abs(out[:half] - np.sin(angle))) < 2e-4
        assert np.max(np.abs(out[half:] - np.cos(angle))) < 2e-4
    zero = np.zeros(64, np.float32)
    oracle.lib().vo_sinusoid(0.0, 64, oracle.ptr(zero))
    assert np.array_equal(zero, np.concatenate([np.zeros(32), np.ones(32)]).astype(np.float32))


# ---- the DiT against a float64 torch formulation --------------------------------

def torch_dit_velocity(weights, oracle, mu, cond_latent, x, t, bf16_weights=False):
    """The local DiT in float64 torch from its description (no bf16 rounding,
    torch's attention), for comparison at tolerance. `bf16_weights` takes
    every matrix as bf16(scale q) (numpy's rounding of the float64 value)."""
    c = weights.config
    td = torch.float64

    def W(blocks):
        n, kb, _ = blocks.shape
        values = oracle.q8_values(np.ascontiguousarray(blocks), n, kb * 32)
        if bf16_weights:
            values = synth.bf16_values(synth.bf16_bits(values.astype(np.float32))) \
                .astype(np.float64)
        return torch.from_numpy(values)

    def vec(bits):
        return torch.from_numpy(synth.bf16_values(bits).astype(np.float64))

    def proj(name, inp):
        blocks, bias = weights.projections[name]
        return inp @ W(blocks).T + vec(bias)

    def rms(h, g):
        return h / torch.sqrt((h * h).mean(-1, keepdim=True) + c.eps) * vec(g)

    def sinus(tt, width):
        half = width // 2
        freq = torch.exp(-torch.arange(half, dtype=td) * math.log(10000.0) / (half - 1))
        a = 1000.0 * tt * freq
        return torch.cat([torch.sin(a), torch.cos(a)])

    silu = torch.nn.functional.silu
    time = proj("time_2", silu(proj("time_1", sinus(t, c.time_in))))
    if c.has_delta:
        time = time + proj("delta_2", silu(proj("delta_1", sinus(0.0, c.time_in))))
    cond_rows = proj("cond_proj", torch.from_numpy(cond_latent.astype(np.float64)))
    x_rows = proj("in_proj", torch.from_numpy(x.astype(np.float64)))
    mu_t = torch.from_numpy(mu.astype(np.float64)).reshape(2, c.hidden)
    seq = []
    for branch in range(2):
        head = mu_t if branch == 0 else torch.zeros_like(mu_t)
        seq.append(torch.cat([head, time[None], cond_rows, x_rows]))
    h = torch.stack(seq)  # [2][11][hidden]
    length = 3 + 2 * c.patch
    pos = torch.arange(length, dtype=td)
    half = c.head_dim // 2
    factors = torch.tensor(c.rope_factors if c.rope_factors else [1.0] * half, dtype=td)
    inv = c.rope_theta ** (-2.0 * torch.arange(half, dtype=td) / c.head_dim)
    ang = pos[:, None] / factors[None, :] * inv[None, :]
    cos, sin = torch.cos(ang) * c.rope_scaling, torch.sin(ang) * c.rope_scaling

    def rope(v):  # [2][heads][length][hd]
        a, b = v[..., :half], v[..., half:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], -1)

    for layer in weights.layers:
        n1 = rms(h, layer["input_norm"])
        qkv = n1 @ W(layer["qkv"]).T
        qw, kw = c.q_width, c.kv_heads * c.head_dim
        q = qkv[..., :qw].reshape(2, length, c.heads, c.head_dim).transpose(1, 2)
        k = qkv[..., qw:qw + kw].reshape(2, length, c.kv_heads, c.head_dim).transpose(1, 2)
        v = qkv[..., qw + kw:].reshape(2, length, c.kv_heads, c.head_dim).transpose(1, 2)
        q, k = rope(q), rope(k)
        g = c.heads // c.kv_heads
        k, v = k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)
        a = torch.nn.functional.scaled_dot_product_attention(q, k, v)
        a = a.transpose(1, 2).reshape(2, length, qw)
        h = h + a @ W(layer["o"]).T
        n2 = rms(h, layer["post_norm"])
        gu = n2 @ W(layer["gate_up"]).T
        act = silu(gu[..., :c.ffn]) * gu[..., c.ffn:]
        h = h + act @ W(layer["down"]).T
    out = rms(h, weights.norm)[:, 3 + c.patch:]  # [2][patch][hidden]
    return proj("out_proj", out).numpy()


@pytest.mark.parametrize("config", [
    synth.DitConfig(hidden=256, heads=4, kv_heads=4, head_dim=64, ffn=512,
                    layers=2, time_in=128),
    synth.DitConfig(hidden=256, heads=4, kv_heads=2, head_dim=128, ffn=512,
                    layers=2, time_in=256, has_delta=True, eps=1e-5,
                    rope_factors=synth.VOXCPM2_SHORT_FACTORS),
], ids=["mha-hd64", "gqa-hd128-delta"])
@pytest.mark.parametrize("bf16_weights", [False, True], ids=["q8", "bf16-weights"])
def test_dit_velocity_against_float64_torch(oracle, config, bf16_weights):
    rope = oracle.rope_table(config.rope_theta, config.head_dim, config.rope_factors,
                             config.rope_scaling, 3 + 2 * config.patch)
    weights = synth.dit_weights(config, 11, rope)
    inputs = synth.patch_inputs(config, 12)
    dit = oracle.OracleDit(weights, bf16_weights=bf16_weights)
    got = dit.velocity(inputs.mu, inputs.cond_latent, inputs.noise, 0.63)
    ref = torch_dit_velocity(weights, oracle, inputs.mu, inputs.cond_latent,
                             inputs.noise, 0.63, bf16_weights=bf16_weights)
    error = np.linalg.norm(got - ref) / np.linalg.norm(ref)
    assert error < 1e-2, error  # bf16 activations against float64
    # A planted slip in the oracle's composition (swapping the CFG branches)
    # fails the same bound.
    assert np.linalg.norm(got[::-1] - ref) / np.linalg.norm(ref) > 5e-2
    if bf16_weights:
        # The bf16 matrices are really the ones multiplied: the result moves
        # off the Q8_0 one by the weights' rounding, and only by that.
        q8 = oracle.OracleDit(weights).velocity(inputs.mu, inputs.cond_latent,
                                                inputs.noise, 0.63)
        moved = np.linalg.norm(got - q8) / np.linalg.norm(q8)
        assert 1e-6 < moved < 2e-2, moved


def test_dit_patch_composes_evaluations(oracle):
    """The sampler equals its steps: cond rows and time vectors, then
    eval + guided Euler per evaluated step."""
    config = synth.DitConfig(hidden=128, heads=2, kv_heads=1, head_dim=64, ffn=256,
                             layers=1, time_in=128, has_delta=True)
    rope = oracle.rope_table(10000.0, 64, None, 1.0, 11)
    weights = synth.dit_weights(config, 13, rope)
    inputs = synth.patch_inputs(config, 14)
    dit = oracle.OracleDit(weights, threads=2)
    t, dt, ev = oracle.euler_schedule(5, 1.0, True)
    got = dit.patch(inputs.mu, inputs.cond_latent, inputs.noise, t, dt, ev, 2.0, True)
    x = inputs.noise.copy()
    cond = dit.cond_rows(inputs.cond_latent)
    for step in range(5):
        if not ev[step]:
            continue
        v = dit.eval(inputs.mu, cond, x, dit.time_vector(float(t[step])))
        flat = np.ascontiguousarray(v.reshape(-1))
        oracle.lib().vo_guided_euler(oracle.ptr(flat), oracle.ptr(x), x.size, 2.0,
                                     float(dt[step]), 1)
    assert np.array_equal(got, x)


# ---- a stack with a key/value cache against a float64 torch formulation ----

def torch_stack(weights, oracle, rope, hidden, sequences, causal):
    """The MiniCPM4 stack in float64 torch from its description over whole
    sequences (no cache: every key of a sequence at once, torch's attention
    with its own causal mask). hidden [S][T][hidden] float; returns
    (residual stream after the layers, final norm's output)."""
    c = weights.config
    td = torch.float64

    def W(blocks):
        n, kb, _ = blocks.shape
        return torch.from_numpy(oracle.q8_values(np.ascontiguousarray(blocks), n, kb * 32))

    def vec(bits):
        return torch.from_numpy(synth.bf16_values(bits).astype(np.float64))

    def rms(h, g):
        return h / torch.sqrt((h * h).mean(-1, keepdim=True) + c.eps) * vec(g)

    h = torch.from_numpy(hidden.astype(np.float64)).reshape(sequences, -1, c.hidden)
    length = h.shape[1]
    half = c.head_dim // 2
    if rope is not None:
        table = torch.from_numpy(rope[:length].astype(np.float64))
        cos, sin = table[:, :half], table[:, half:]

    def rotate(v):
        if rope is None:
            return v
        a, b = v[..., :half], v[..., half:]
        return torch.cat([a * cos - b * sin, b * cos + a * sin], -1)

    for layer in weights.layers:
        qkv = rms(h, layer["input_norm"]) @ W(layer["qkv"]).T
        qw, kw = c.q_width, c.kv_heads * c.head_dim
        q = qkv[..., :qw].reshape(sequences, length, c.heads, c.head_dim).transpose(1, 2)
        k = qkv[..., qw:qw + kw].reshape(sequences, length, c.kv_heads, c.head_dim).transpose(1, 2)
        v = qkv[..., qw + kw:].reshape(sequences, length, c.kv_heads, c.head_dim).transpose(1, 2)
        q, k = rotate(q), rotate(k)
        g = c.heads // c.kv_heads
        k, v = k.repeat_interleave(g, 1), v.repeat_interleave(g, 1)
        a = torch.nn.functional.scaled_dot_product_attention(q, k, v, is_causal=causal)
        h = h + a.transpose(1, 2).reshape(sequences, length, qw) @ W(layer["o"]).T
        gu = rms(h, layer["post_norm"]) @ W(layer["gate_up"]).T
        h = h + (torch.nn.functional.silu(gu[..., :c.ffn]) * gu[..., c.ffn:]) @ W(layer["down"]).T
    return h.reshape(-1, c.hidden).numpy(), rms(h, weights.norm).reshape(-1, c.hidden).numpy()


def relative(a, b):
    return float(np.linalg.norm(np.asarray(a, np.float64) - b) / np.linalg.norm(b))


STACK_CONFIGS = [
    synth.StackConfig(hidden=256, heads=4, kv_heads=2, head_dim=64, ffn=512, layers=2,
                      rope_factors=tuple(1.0 + 0.1 * i for i in range(32))),
    synth.StackConfig(hidden=128, heads=2, kv_heads=1, head_dim=64, ffn=256, layers=2,
                      rope=False),
]


@pytest.mark.parametrize("config", STACK_CONFIGS, ids=["gqa-rope", "no-rope"])
def test_stack_incremental_decode_equals_full_causal_forward(oracle, config):
    """A causal prefill of 6 rows, then 3 one-row steps through the cache
    (the LM's decode: positions = cache rows = past), equal row for row the
    whole 9-row causal sequence in float64 torch."""
    rope = oracle.rope_table(config.rope_theta, config.head_dim, config.rope_factors,
                             config.rope_scaling, 16) if config.rope else None
    weights = synth.stack_weights(config, 21)
    stack = oracle.OracleStack(weights, rope, threads=4)
    rng = synth.Rng(22, 1)
    total, prefix, capacity = 9, 6, 12
    h0 = rng.normal(total * config.hidden).astype(np.float32).reshape(total, config.hidden)
    ref_h, ref_out = torch_stack(weights, oracle, rope, h0, 1, True)
    shape = (config.layers, config.kv_heads, capacity, config.head_dim)
    k_cache, v_cache = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    rows = np.arange(prefix, dtype=np.int32)
    h, out = stack.forward(h0[:prefix], rows, rows, prefix, prefix, 0, True, k_cache, v_cache)
    assert relative(out, ref_out[:prefix]) < 5e-4
    assert relative(h, ref_h[:prefix]) < 5e-4
    for position in range(prefix, total):
        at = np.array([position], np.int32)
        h, out = stack.forward(h0[position:position + 1], at, at, 1, 1, position, True,
                               k_cache, v_cache)
        assert relative(out, ref_out[position:position + 1]) < 5e-4, position
        assert relative(h, ref_h[position:position + 1]) < 5e-4, position
    # A planted slip: the last step attending one key short (past - 1)
    # moves the output well past the bound (bf16 activations against
    # float64 stay near 1e-4).
    kc, vc = k_cache.copy(), v_cache.copy()
    at = np.array([total - 1], np.int32)
    _, bad = stack.forward(h0[total - 1:], at, at, 1, 1, total - 2, True, kc, vc)
    assert relative(bad, ref_out[total - 1:]) > 2e-3


def test_stack_bidirectional_sequences(oracle):
    """The local encoder's layout: two 5-row sequences attending within
    themselves, non-causal, rotary positions row % 5, against float64 torch;
    swapping the two sequences' rows moves every output."""
    config = STACK_CONFIGS[0]
    rope = oracle.rope_table(config.rope_theta, config.head_dim, config.rope_factors,
                             config.rope_scaling, 8)
    weights = synth.stack_weights(config, 23)
    stack = oracle.OracleStack(weights, rope, threads=4)
    rng = synth.Rng(24, 1)
    h0 = rng.normal(10 * config.hidden).astype(np.float32).reshape(10, config.hidden)
    ref_h, ref_out = torch_stack(weights, oracle, rope, h0, 2, False)
    shape = (config.layers, config.kv_heads, 10, config.head_dim)
    k_cache, v_cache = np.zeros(shape, np.float32), np.zeros(shape, np.float32)
    positions = (np.arange(10) % 5).astype(np.int32)
    h, out = stack.forward(h0, positions, np.arange(10, dtype=np.int32), 5, 5, 0, False,
                           k_cache, v_cache)
    assert relative(out, ref_out) < 5e-4
    assert relative(h, ref_h) < 5e-4
    assert relative(out[::-1], ref_out) > 5e-2


# ---- AudioVAE's decoder against a float64 torch formulation ----------------

def torch_vae_decode(weights, latents):
    """AudioVAE V2's causal decoder in float64 torch from the module
    description: causal convolutions as left-padded conv1d, the causal
    transposed convolution as conv_transpose1d's first T s outputs, Snake
    x + sin^2(a x) / (a + 1e-9), the output conv's tanh."""
    t = weights.tensors
    F = torch.nn.functional

    def T(a):
        return torch.from_numpy(np.asarray(a, dtype=np.float64))

    def snake(x, a):
        a = T(a)[None, :, None]
        return x + torch.sin(a * x) ** 2 / (a + 1e-9)

    def depthwise(x, w, b, d):
        c = x.shape[1]
        return F.conv1d(F.pad(x, (6 * d, 0)), T(w).reshape(c, 1, 7), T(b), dilation=d, groups=c)

    x = T(latents).T[None]  # [1][latent][frames]
    x = depthwise(x, t["in_depthwise"], t["in_depthwise_bias"], 1)
    x = F.conv1d(x, T(t["in_pointwise"])[:, :, None], T(t["in_pointwise_bias"]))
    for block in t["blocks"]:
        s = block["stride"]
        frames = x.shape[2]
        x = x * T(block["scale"])[None, :, None] + T(block["bias"])[None, :, None]
        x = snake(x, block["alpha"])
        x = F.conv_transpose1d(x, T(block["up"]), T(block["up_bias"]), stride=s)[..., :frames * s]
        for unit, d in zip(block["units"], (1, 3, 9)):
            y = snake(x, unit["alpha_in"])
            y = depthwise(y, unit["depthwise"], unit["depthwise_bias"], d)
            y = snake(y, unit["alpha_out"])
            x = x + F.conv1d(y, T(unit["pointwise"])[:, :, None], T(unit["pointwise_bias"]))
    x = snake(x, t["out_alpha"])
    c = x.shape[1]
    x = F.conv1d(F.pad(x, (6, 0)), T(t["out_conv"]).reshape(1, c, 7), T([t["out_bias"]]))
    return torch.tanh(x)[0, 0].numpy()


def test_vae_decoder_against_float64_torch(oracle):
    config = synth.VaeConfig(latent=16, decoder_dim=64, rates=(3, 2, 2))
    weights = synth.vae_weights(config, 81)
    vae = oracle.OracleVae(weights)
    rng = synth.Rng(82, 1)
    latents = rng.normal(9 * config.latent).astype(np.float32).reshape(9, config.latent)
    got = vae.decode(latents)
    ref = torch_vae_decode(weights, latents)
    assert got.shape == ref.shape == (9 * config.hop,)
    error = float(np.max(np.abs(got - ref)))
    assert error < 2e-5, error  # float32 against float64
    assert np.std(ref) > 0.05  # a signal, not a saturated or silent output
    # Causality: the first five frames' samples do not depend on the rest.
    head = vae.decode(latents[:5])
    assert np.array_equal(head, got[:5 * config.hop])
    # A planted slip (the transposed convolution's previous-frame taps taken
    # from the current frame) is caught.
    slip = synth.VaeWeightsHost(config, dict(weights.tensors))
    blocks = [dict(b) for b in weights.tensors["blocks"]]
    s = blocks[0]["stride"]
    up = blocks[0]["up"].copy()
    up[:, :, s:] = up[:, :, :s]
    blocks[0]["up"] = up
    slip.tensors["blocks"] = blocks
    assert np.max(np.abs(oracle.OracleVae(slip).decode(latents) - ref)) > 1e-2
