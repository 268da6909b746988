"""Seeded synthetic inputs of the DiT hot path's workloads.

A self-specified generator (splitmix64 counters, Box-Muller in double) so
that the same seed gives the same values on every machine and numpy
version. The laws follow the workloads: Q8_0 weights with int8 uniform in
[-127, 127] and float16 scales fp16_rne(|N(0, 0.02)| / 127) (subnormals
kept), bf16 activations ~ N(0, 1), norm weights bf16(1 + N(0, 0.02)),
biases bf16(N(0, 0.02)).
"""
from __future__ import annotations

import dataclasses

import numpy as np

_GOLDEN = np.uint64(0x9E3779B97F4A7C15)
_M1 = np.uint64(0xBF58476D1CE4E5B9)
_M2 = np.uint64(0x94D049BB133111EB)


def _mix(z: np.ndarray) -> np.ndarray:
    with np.errstate(over="ignore"):
        z = (z ^ (z >> np.uint64(30))) * _M1
        z = (z ^ (z >> np.uint64(27))) * _M2
    return z ^ (z >> np.uint64(31))


class Rng:
    """splitmix64 counter stream: value i is mix(key + (i + 1) * golden)."""

    def __init__(self, seed: int, stream: int = 0):
        key = _mix(np.array([seed & 0xFFFFFFFFFFFFFFFF], dtype=np.uint64))[0]
        with np.errstate(over="ignore"):
            self.key = _mix(np.array([key ^ np.uint64(stream * 0x2545F491)],
                                     dtype=np.uint64))[0]
        self.counter = 0

    def bits(self, count: int) -> np.ndarray:
        index = np.arange(self.counter + 1, self.counter + count + 1,
                          dtype=np.uint64)
        self.counter += count
        with np.errstate(over="ignore"):
            return _mix(self.key + index * _GOLDEN)

    def uniform(self, count: int) -> np.ndarray:
        """Doubles in [0, 1)."""
        return (self.bits(count) >> np.uint64(11)).astype(np.float64) * 2.0**-53

    def normal(self, count: int, std: float = 1.0) -> np.ndarray:
        pairs = (count + 1) // 2
        u1 = self.uniform(pairs)
        u2 = self.uniform(pairs)
        radius = np.sqrt(-2.0 * np.log1p(-u1))
        angle = 2.0 * np.pi * u2
        values = np.empty(2 * pairs)
        values[0::2] = radius * np.cos(angle)
        values[1::2] = radius * np.sin(angle)
        return values[:count] * std

    def int8(self, count: int) -> np.ndarray:
        """Uniform in [-127, 127]."""
        return ((self.bits(count) % np.uint64(255)).astype(np.int64) - 127).astype(np.int8)


def bf16_bits(values) -> np.ndarray:
    """float32 -> bfloat16 bits (uint16), round to nearest even, NaN quiet."""
    f = np.ascontiguousarray(values, dtype=np.float32)
    bits = f.view(np.uint32).astype(np.uint64)
    rounded = ((bits + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    nan = np.isnan(f)
    if nan.any():
        rounded[nan] = ((bits[nan] >> 16) | 0x40).astype(np.uint16)
    return rounded


def bf16_values(bits: np.ndarray) -> np.ndarray:
    return (bits.astype(np.uint32) << 16).view(np.float32)


def q8_blocks(rng: Rng, n: int, k: int) -> np.ndarray:
    """GGML Q8_0 blocks [n][k/32][34] (uint8): fp16 LE scale, 32 int8."""
    assert k % 32 == 0
    count = n * (k // 32)
    scales = (np.abs(rng.normal(count, 0.02)) / 127.0).astype(np.float32)
    scale_bits = scales.astype(np.float16).view(np.uint16)
    q = rng.int8(count * 32).reshape(count, 32)
    blocks = np.empty((count, 34), dtype=np.uint8)
    blocks[:, 0] = (scale_bits & 0xFF).astype(np.uint8)
    blocks[:, 1] = (scale_bits >> 8).astype(np.uint8)
    blocks[:, 2:] = q.view(np.uint8)
    return blocks.reshape(n, k // 32, 34)


def activations(rng: Rng, rows: int, width: int) -> np.ndarray:
    """bf16 bits [rows][width] ~ N(0, 1)."""
    return bf16_bits(rng.normal(rows * width).astype(np.float32)).reshape(rows, width)


def bf16_vector(rng: Rng, count: int, mean: float, std: float) -> np.ndarray:
    return bf16_bits((mean + rng.normal(count, std)).astype(np.float32))


@dataclasses.dataclass(frozen=True)
class DitConfig:
    """A local-DiT shape (vx_dit_shape) with its sampler settings."""
    hidden: int = 1024
    heads: int = 16
    kv_heads: int = 16
    head_dim: int = 64
    ffn: int = 4096
    layers: int = 12
    patch: int = 4
    feat: int = 64
    time_in: int = 256
    has_delta: bool = False
    eps: float = 1e-6
    rope_theta: float = 10000.0
    rope_factors: tuple | None = None  # head_dim / 2 LongRoPE factors
    rope_scaling: float = 1.0
    steps: int = 10
    sway: float = 0.0
    skip: bool = False      # CFG-Zero*'s zero-velocity first steps
    zero_star: bool = False  # CFG-Zero*'s guidance scale
    cfg: float = 2.0

    @property
    def rows(self) -> int:
        return 2 * (3 + 2 * self.patch)

    @property
    def q_width(self) -> int:
        return self.heads * self.head_dim

    @property
    def qkv_width(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


# The synthetic DiT of the per-patch workload: 12 blocks of hidden 1024,
# 16 heads x 64, SwiGLU 4096, eps 1e-6, RoPE base 10000, time 256 -> 1024,
# 10 uniform Euler steps with plain CFG 2.0.
SYNTHETIC_DIT = DitConfig()

# The released VoxCPM2 local DiT (tests/config_samples.hpp:176-189 of the
# reference; config.cpp:144-154): 16 q heads x 128 with 2 KV heads, eps
# 1e-5, LongRoPE short factors (scale 1.0), time embedding 1024 with the
# delta term, sway-sampled schedule, CFG-Zero*.
VOXCPM2_SHORT_FACTORS = (
    0.9977997200264581, 1.014658295992452, 1.0349680404997148,
    1.059429246056193, 1.0888815016813513, 1.1243301355211495,
    1.166977103606075, 1.2182568066927284, 1.2798772354275727,
    1.3538666751582975, 1.4426259039919596, 1.5489853358570191,
    1.6762658237220625, 1.8283407612492941, 2.0096956085876183,
    2.225478927469756, 2.481536379650452, 2.784415934557119,
    3.1413289096347365, 3.560047844772632, 4.048719380066383,
    4.615569542115128, 5.2684819496549835, 6.014438591970396,
    6.858830049237097, 7.804668263503327, 8.851768731513417,
    9.99600492938444, 11.228766118181639, 12.536757560834843,
    13.902257701387796, 15.303885189125953, 16.717837610115794,
    18.119465097853947, 19.484965238406907, 20.792956681060105,
    22.02571786985731, 23.16995406772833, 24.217054535738416,
    25.16289275000465, 26.007284207271347, 26.753240849586767,
    27.40615325712662, 27.973003419175363, 28.461674954469114,
    28.880393889607006, 29.237306864684626, 29.540186419591297,
    29.79624387177199, 30.01202719065413, 30.193382037992453,
    30.34545697551969, 30.47273746338473, 30.579096895249787,
    30.66785612408345, 30.741845563814174, 30.80346599254902,
    30.85474569563567, 30.897392663720595, 30.932841297560394,
    30.962293553185553, 30.986754758742034, 31.007064503249293,
    31.02392307921529,
)
VOXCPM2_DIT = DitConfig(
    heads=16, kv_heads=2, head_dim=128, eps=1e-5, time_in=1024,
    has_delta=True, rope_factors=VOXCPM2_SHORT_FACTORS, rope_scaling=1.0,
    sway=1.0, skip=True, zero_star=True)


@dataclasses.dataclass
class DitWeightsHost:
    """Host copies of a DiT's weights: GGML Q8_0 blocks and bf16 vectors."""
    config: DitConfig
    layers: list  # dicts: input_norm, qkv, o, post_norm, gate_up, down
    norm: np.ndarray
    projections: dict  # name -> (blocks, bias bits)
    rope: np.ndarray | None


PROJECTIONS = ("in_proj", "cond_proj", "out_proj", "time_1", "time_2",
               "delta_1", "delta_2")


def projection_shape(config: DitConfig, name: str) -> tuple[int, int]:
    """(out, in) of a projection."""
    return {
        "in_proj": (config.hidden, config.feat),
        "cond_proj": (config.hidden, config.feat),
        "out_proj": (config.feat, config.hidden),
        "time_1": (config.hidden, config.time_in),
        "time_2": (config.hidden, config.hidden),
        "delta_1": (config.hidden, config.time_in),
        "delta_2": (config.hidden, config.hidden),
    }[name]


def dit_weights(config: DitConfig, seed: int, rope: np.ndarray | None = None
                ) -> DitWeightsHost:
    rng = Rng(seed, 1)
    layers = []
    h = config.hidden
    for _ in range(config.layers):
        layers.append({
            "input_norm": bf16_vector(rng, h, 1.0, 0.02),
            "qkv": q8_blocks(rng, config.qkv_width, h),
            "o": q8_blocks(rng, h, config.q_width),
            "post_norm": bf16_vector(rng, h, 1.0, 0.02),
            "gate_up": q8_blocks(rng, 2 * config.ffn, h),
            "down": q8_blocks(rng, h, config.ffn),
        })
    norm = bf16_vector(rng, h, 1.0, 0.02)
    projections = {}
    for name in PROJECTIONS:
        if name.startswith("delta") and not config.has_delta:
            continue
        out, inp = projection_shape(config, name)
        projections[name] = (q8_blocks(rng, out, inp),
                             bf16_vector(rng, out, 0.0, 0.02))
    return DitWeightsHost(config, layers, norm, projections, rope)


@dataclasses.dataclass
class PatchInputs:
    mu: np.ndarray           # float32 [2 hidden], bf16-representable
    cond_latent: np.ndarray  # float32 [patch][feat], bf16-representable
    noise: np.ndarray        # float32 [patch][feat]


def patch_inputs(config: DitConfig, seed: int) -> PatchInputs:
    rng = Rng(seed, 2)
    mu = bf16_values(bf16_bits(rng.normal(2 * config.hidden).astype(np.float32)))
    cond = bf16_values(bf16_bits(
        rng.normal(config.patch * config.feat).astype(np.float32)))
    noise = rng.normal(config.patch * config.feat).astype(np.float32)
    return PatchInputs(mu.copy(), cond.reshape(config.patch, config.feat).copy(),
                       noise.reshape(config.patch, config.feat))


@dataclasses.dataclass(frozen=True)
class StackConfig:
    """A MiniCPM4 stack with a key/value cache (vx_stack_shape): the LMs
    and the local encoder (config.hpp:15-31)."""
    hidden: int = 2048
    heads: int = 16
    kv_heads: int = 2
    head_dim: int = 128
    ffn: int = 6144
    layers: int = 28
    eps: float = 1e-5
    rope: bool = True
    rope_theta: float = 10000.0
    rope_factors: tuple | None = None
    rope_scaling: float = 1.0

    @property
    def q_width(self) -> int:
        return self.heads * self.head_dim

    @property
    def qkv_width(self) -> int:
        return (self.heads + 2 * self.kv_heads) * self.head_dim


# VoxCPM2's stacks (tests/config_samples.hpp of the reference): the base LM
# (28 layers, hidden 2048, MLP 6144, 16 q heads x 128 with 2 KV heads,
# LongRoPE), the residual LM (8 layers, no rotary embedding) and the local
# encoder (12 layers, hidden 1024, MLP 4096, heads as the LM's).
VOXCPM2_BASE_LM = StackConfig(rope_factors=VOXCPM2_SHORT_FACTORS)
VOXCPM2_RESIDUAL_LM = StackConfig(layers=8, rope=False)
VOXCPM2_ENCODER = StackConfig(hidden=1024, ffn=4096, layers=12,
                              rope_factors=VOXCPM2_SHORT_FACTORS)


@dataclasses.dataclass
class StackWeightsHost:
    """Host copies of a stack's weights: GGML Q8_0 blocks and bf16 vectors."""
    config: StackConfig
    layers: list  # dicts: input_norm, qkv, o, post_norm, gate_up, down
    norm: np.ndarray


def stack_weights(config: StackConfig, seed: int) -> StackWeightsHost:
    rng = Rng(seed, 3)
    layers = []
    h = config.hidden
    for _ in range(config.layers):
        layers.append({
            "input_norm": bf16_vector(rng, h, 1.0, 0.02),
            "qkv": q8_blocks(rng, config.qkv_width, h),
            "o": q8_blocks(rng, h, config.q_width),
            "post_norm": bf16_vector(rng, h, 1.0, 0.02),
            "gate_up": q8_blocks(rng, 2 * config.ffn, h),
            "down": q8_blocks(rng, h, config.ffn),
        })
    return StackWeightsHost(config, layers, bf16_vector(rng, h, 1.0, 0.02))


@dataclasses.dataclass(frozen=True)
class VaeConfig:
    """AudioVAE V2's decoder shape (AudioVaeConfig, config.hpp:55-72)."""
    latent: int = 64
    decoder_dim: int = 2048
    rates: tuple = (8, 6, 5, 2, 2, 2)

    @property
    def hop(self) -> int:
        return int(np.prod(self.rates))

    def channels(self, block: int) -> tuple[int, int]:
        """(in, out) channels of decoder block `block`."""
        c = self.decoder_dim >> block
        return c, c // 2


# VoxCPM2's AudioVAE (tests/config_samples.hpp of the reference): latent 64,
# decoder 2048 channels, rates 8 6 5 2 2 2 (1920 samples per latent frame at
# 48 kHz).
VOXCPM2_VAE = VaeConfig()


@dataclasses.dataclass
class VaeWeightsHost:
    """float32 decoder weights in PyTorch's layouts, weight norm folded;
    blocks: dicts scale, bias, alpha, up [in][out][2s], up_bias, units
    (dicts alpha_in, depthwise [c][7], depthwise_bias, alpha_out,
    pointwise [c][c], pointwise_bias)."""
    config: VaeConfig
    tensors: dict


def vae_weights(config: VaeConfig, seed: int) -> VaeWeightsHost:
    """Random decoder weights scaled by 1/sqrt(fan-in) (activations stay
    O(1) through the blocks); Snake alphas 1 + N(0, 0.1) kept positive."""
    rng = Rng(seed, 5)

    def normal(shape, std):
        count = int(np.prod(shape))
        return (rng.normal(count) * std).astype(np.float32).reshape(shape)

    def alpha(c):
        return np.abs(1.0 + normal((c,), 0.1)).astype(np.float32) + 0.05

    t = {"in_depthwise": normal((config.latent, 7), 1 / np.sqrt(7)),
         "in_depthwise_bias": normal((config.latent,), 0.02),
         "in_pointwise": normal((config.decoder_dim, config.latent), 1 / np.sqrt(config.latent)),
         "in_pointwise_bias": normal((config.decoder_dim,), 0.02), "blocks": []}
    for b, s in enumerate(config.rates):
        c_in, c_out = config.channels(b)
        units = []
        for _ in range(3):
            units.append({"alpha_in": alpha(c_out),
                          "depthwise": normal((c_out, 7), 1 / np.sqrt(7)),
                          "depthwise_bias": normal((c_out,), 0.02),
                          "alpha_out": alpha(c_out),
                          "pointwise": normal((c_out, c_out), 0.5 / np.sqrt(c_out)),
                          "pointwise_bias": normal((c_out,), 0.02)})
        t["blocks"].append({"stride": s, "scale": 1.0 + normal((c_in,), 0.05),
                            "bias": normal((c_in,), 0.05), "alpha": alpha(c_in),
                            "up": normal((c_in, c_out, 2 * s), 1 / np.sqrt(2 * c_in)),
                            "up_bias": normal((c_out,), 0.02), "units": units})
    c_last = config.channels(len(config.rates) - 1)[1]
    t["out_alpha"] = alpha(c_last)
    t["out_conv"] = normal((c_last, 7), 1 / np.sqrt(7 * c_last))
    t["out_bias"] = float(normal((1,), 0.02)[0])
    return VaeWeightsHost(config, t)
