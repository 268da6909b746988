"""ctypes binding of the CPU oracle (oracle/liboracle.so) -- test
infrastructure: the checker the GPU results are compared against, and the
timed CPU baseline. Builds the library with make when it is missing.
"""
from __future__ import annotations

import ctypes
import pathlib
import subprocess

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[1]
ORACLE_DIR = ROOT / "oracle"
LIBRARY = ORACLE_DIR / "liboracle.so"

c_size = ctypes.c_size_t
c_int = ctypes.c_int
c_float = ctypes.c_float
c_void_p = ctypes.c_void_p


class Projection(ctypes.Structure):
    _fields_ = [("weight", c_void_p), ("bias", c_void_p)]


class Layer(ctypes.Structure):
    _fields_ = [("input_norm", c_void_p), ("qkv", c_void_p), ("o", c_void_p),
                ("post_norm", c_void_p), ("gate_up", c_void_p),
                ("down", c_void_p)]


class Dit(ctypes.Structure):
    _fields_ = [(name, c_size) for name in (
        "hidden", "heads", "kv_heads", "head_dim", "ffn", "layers", "patch",
        "feat", "time_in")] + [
        ("eps", c_float), ("has_delta", c_int), ("rope", c_void_p),
        ("layer", ctypes.POINTER(Layer)), ("norm", c_void_p),
        ("in_proj", Projection), ("cond_proj", Projection),
        ("out_proj", Projection), ("time_1", Projection),
        ("time_2", Projection), ("delta_1", Projection),
        ("delta_2", Projection), ("threads", c_int), ("bf16_weights", c_int)]


_SIGNATURES = {
    "vo_bf16_bits": ([c_float], ctypes.c_uint16),
    "vo_bf16_value": ([ctypes.c_uint16], c_float),
    "vo_half_value": ([ctypes.c_uint16], c_float),
    "vo_half_bits": ([c_float], ctypes.c_uint16),
    "vo_bf16_round_array": ([c_void_p, c_void_p, c_size], None),
    "vo_q8_dequant_bf16": ([c_void_p, c_size, c_size, c_void_p], None),
    "vo_q8_values": ([c_void_p, c_size, c_size, c_void_p], None),
    "vo_q8_linear": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                      c_int, c_int], None),
    "vo_q8_check": ([c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size,
                     c_size], ctypes.c_double),
    "vo_bf16_linear": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size, c_int,
                        c_int], None),
    "vo_bf16_check": ([c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size,
                       c_size], ctypes.c_double),
    "vo_rms_norm": ([c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size,
                     c_float], None),
    "vo_rope_table": ([ctypes.c_double, c_size, c_void_p, c_float, c_size,
                       c_void_p], None),
    "vo_qkv_rope": ([c_void_p] * 7 + [c_size] * 5, None),
    "vo_attention": ([c_void_p] * 4 + [c_size] * 4 + [c_int] + [c_size] * 4,
                     None),
    "vo_swiglu": ([c_void_p, c_void_p, c_size, c_size], None),
    "vo_add_bias": ([c_void_p, c_void_p, c_size, c_size], None),
    "vo_to_bf16": ([c_void_p, c_void_p, c_size, c_int], None),
    "vo_gather_rows": ([c_void_p, c_void_p, c_void_p, c_size, c_size], None),
    "vo_assemble_dit": ([c_void_p] * 5 + [c_size, c_size], None),
    "vo_guided_euler": ([c_void_p, c_void_p, c_size, c_float, c_float, c_int],
                        None),
    "vo_linspace": ([c_float, c_float, c_size, c_void_p], None),
    "vo_euler_schedule": ([c_size, c_float, c_int, c_void_p, c_void_p,
                           c_void_p], None),
    "vo_sinusoid": ([c_float, c_size, c_void_p], None),
    "vo_dit_time_vector": ([ctypes.POINTER(Dit), c_float, c_void_p], None),
    "vo_dit_cond_rows": ([ctypes.POINTER(Dit), c_void_p, c_void_p], None),
    "vo_dit_eval": ([ctypes.POINTER(Dit)] + [c_void_p] * 5, None),
    "vo_dit_velocity": ([ctypes.POINTER(Dit), c_void_p, c_void_p, c_void_p,
                         c_float, c_void_p], None),
    "vo_dit_patch": ([ctypes.POINTER(Dit), c_void_p, c_void_p, c_void_p,
                      c_void_p, c_void_p, c_void_p, c_size, c_float, c_int],
                     None),
    # (vo_stack*, hidden, output, rows, positions, cache_rows,
    #  rows_per_sequence, keys_per_sequence, past, causal, k, v, capacity)
    "vo_vae_decode": ([c_void_p, c_void_p, c_size, c_void_p], None),
    "vo_stack_forward": ([c_void_p, c_void_p, c_void_p, c_size, c_void_p, c_void_p,
                          c_size, c_size, c_size, c_int, c_void_p, c_void_p, c_size],
                         None),
}

_lib = None


def build() -> pathlib.Path:
    subprocess.run(["make", "-C", str(ORACLE_DIR), "-B", "liboracle.so"],
                   check=True, capture_output=True)
    return LIBRARY


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            build()
        handle = ctypes.CDLL(str(LIBRARY))
        for name, (args, result) in _SIGNATURES.items():
            fn = getattr(handle, name)
            fn.argtypes = args
            fn.restype = result
        _lib = handle
    return _lib


def ptr(array: np.ndarray | None):
    if array is None:
        return None
    assert array.flags["C_CONTIGUOUS"], "oracle arrays must be contiguous"
    return array.ctypes.data


# ---- convenience wrappers ---------------------------------------------------

def q8_dequant_bf16(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    out = np.zeros((n, k), dtype=np.uint16)
    lib().vo_q8_dequant_bf16(ptr(blocks), n, k, ptr(out))
    return out


def q8_values(blocks: np.ndarray, n: int, k: int) -> np.ndarray:
    out = np.zeros((n, k), dtype=np.float64)
    lib().vo_q8_values(ptr(blocks), n, k, ptr(out))
    return out


def q8_linear(x: np.ndarray, blocks: np.ndarray, n: int,
              before: np.ndarray | None = None, threads: int = 8) -> np.ndarray:
    m, k = x.shape
    y = np.zeros((m, n), dtype=np.float32) if before is None else before.copy()
    lib().vo_q8_linear(ptr(x), ptr(blocks), ptr(y), m, k, n,
                       int(before is not None), threads)
    return y


def q8_check(y: np.ndarray, x: np.ndarray, blocks: np.ndarray,
             before: np.ndarray | None = None) -> float:
    m, k = x.shape
    n = y.shape[1]
    y = np.ascontiguousarray(y, dtype=np.float32)
    return lib().vo_q8_check(ptr(y), ptr(x), ptr(blocks), ptr(before), m, k, n)


def bf16_linear(x: np.ndarray, w: np.ndarray, before: np.ndarray | None = None,
                threads: int = 8) -> np.ndarray:
    """x bf16 bits [m][k], w bf16 bits [n][k] -> float32 [m][n]."""
    m, k = x.shape
    n = w.shape[0]
    y = np.zeros((m, n), dtype=np.float32) if before is None else before.copy()
    lib().vo_bf16_linear(ptr(x), ptr(w), ptr(y), m, k, n, int(before is not None), threads)
    return y


def bf16_check(y: np.ndarray, x: np.ndarray, w: np.ndarray,
               before: np.ndarray | None = None) -> float:
    m, k = x.shape
    n = w.shape[0]
    y = np.ascontiguousarray(y, dtype=np.float32)
    return lib().vo_bf16_check(ptr(y), ptr(x), ptr(w), ptr(before), m, k, n)


def euler_schedule(timesteps: int, sway: float, skip: bool):
    t = np.zeros(timesteps, dtype=np.float32)
    dt = np.zeros(timesteps, dtype=np.float32)
    ev = np.zeros(timesteps, dtype=np.int32)
    lib().vo_euler_schedule(timesteps, sway, int(skip), ptr(t), ptr(dt), ptr(ev))
    return t, dt, ev


def rope_table(theta: float, dim: int, factors, scaling: float,
               positions: int) -> np.ndarray:
    table = np.zeros((positions, dim), dtype=np.float32)
    f = None if factors is None else np.ascontiguousarray(factors, dtype=np.float64)
    lib().vo_rope_table(theta, dim, ptr(f), scaling, positions, ptr(table))
    return table


class Stack(ctypes.Structure):
    _fields_ = [(name, c_size) for name in (
        "hidden", "heads", "kv_heads", "head_dim", "ffn", "layers")] + [
        ("eps", ctypes.c_float), ("rope", c_void_p), ("layer", ctypes.POINTER(Layer)),
        ("norm", c_void_p), ("threads", ctypes.c_int), ("bf16_weights", ctypes.c_int)]


class VaeUnit(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("alpha_in", "depthwise", "depthwise_bias",
                                         "alpha_out", "pointwise", "pointwise_bias")]


class VaeBlock(ctypes.Structure):
    _fields_ = [("stride", c_size)] + [(n, c_void_p) for n in (
        "scale", "bias", "alpha", "up", "up_bias")] + [("units", VaeUnit * 3)]


class Vae(ctypes.Structure):
    _fields_ = [(n, c_size) for n in ("latent", "decoder_dim", "block_count")] + [
        (n, c_void_p) for n in ("in_depthwise", "in_depthwise_bias", "in_pointwise",
                                "in_pointwise_bias")] + [
        ("blocks", ctypes.POINTER(VaeBlock)), ("out_alpha", c_void_p),
        ("out_conv", c_void_p), ("out_bias", c_float)]


class OracleDit:
    """A vo_dit over host copies of synthetic weights."""

    def __init__(self, weights, threads: int = 8, bf16_weights: bool = False):
        """`bf16_weights`: every matrix as the bf16 expansion bf16(scale q)
        of its Q8_0 blocks (the reference's bf16 tiles of the same weights)."""
        config = weights.config
        self.config = config
        self._keep = []

        def keep(array):
            array = np.ascontiguousarray(array)
            if bf16_weights and array.ndim == 3 and array.shape[-1] == 34:
                n, blocks, _ = array.shape
                array = q8_dequant_bf16(array, n, blocks * 32)
            self._keep.append(array)
            return array.ctypes.data

        layers = (Layer * config.layers)()
        for index, layer in enumerate(weights.layers):
            layers[index] = Layer(keep(layer["input_norm"]), keep(layer["qkv"]),
                                  keep(layer["o"]), keep(layer["post_norm"]),
                                  keep(layer["gate_up"]), keep(layer["down"]))
        self._layers = layers
        projections = {}
        for name in ("in_proj", "cond_proj", "out_proj", "time_1", "time_2",
                     "delta_1", "delta_2"):
            if name in weights.projections:
                blocks, bias = weights.projections[name]
                projections[name] = Projection(keep(blocks), keep(bias))
            else:
                projections[name] = Projection(None, None)
        rope = None if weights.rope is None else keep(
            np.asarray(weights.rope, dtype=np.float32))
        self.struct = Dit(
            config.hidden, config.heads, config.kv_heads, config.head_dim,
            config.ffn, config.layers, config.patch, config.feat,
            config.time_in, config.eps, int(config.has_delta), rope, layers,
            keep(weights.norm), threads=threads, bf16_weights=int(bf16_weights),
            **projections)

    def time_vector(self, t: float) -> np.ndarray:
        out = np.zeros(self.config.hidden, dtype=np.float32)
        lib().vo_dit_time_vector(ctypes.byref(self.struct), t, ptr(out))
        return out

    def cond_rows(self, cond_latent: np.ndarray) -> np.ndarray:
        out = np.zeros((self.config.patch, self.config.hidden), dtype=np.float32)
        cond = np.ascontiguousarray(cond_latent, np.float32)
        lib().vo_dit_cond_rows(ctypes.byref(self.struct), ptr(cond), ptr(out))
        return out

    def eval(self, mu, cond_rows, x, time_vector) -> np.ndarray:
        out = np.zeros((2, self.config.patch, self.config.feat), dtype=np.float32)
        args = [np.ascontiguousarray(a, dtype=np.float32)
                for a in (mu, cond_rows, x, time_vector)]
        lib().vo_dit_eval(ctypes.byref(self.struct), *map(ptr, args), ptr(out))
        return out

    def velocity(self, mu, cond_latent, x, t: float) -> np.ndarray:
        out = np.zeros((2, self.config.patch, self.config.feat), dtype=np.float32)
        args = [np.ascontiguousarray(a, dtype=np.float32)
                for a in (mu, cond_latent, x)]
        lib().vo_dit_velocity(ctypes.byref(self.struct), *map(ptr, args), t,
                              ptr(out))
        return out

    def patch(self, mu, cond_latent, x, t, dt, evaluate, cfg: float,
              zero_star: bool) -> np.ndarray:
        x = np.array(x, dtype=np.float32, copy=True)
        t = np.ascontiguousarray(t, dtype=np.float32)
        dt = np.ascontiguousarray(dt, dtype=np.float32)
        evaluate = np.ascontiguousarray(evaluate, dtype=np.int32)
        mu = np.ascontiguousarray(mu, np.float32)
        cond = np.ascontiguousarray(cond_latent, np.float32)
        lib().vo_dit_patch(ctypes.byref(self.struct), ptr(mu), ptr(cond),
                           ptr(x), ptr(t), ptr(dt), ptr(evaluate), len(t), cfg,
                           int(zero_star))
        return x


class OracleStack:
    """A vo_stack over host copies of synthetic stack weights."""

    def __init__(self, weights, rope: np.ndarray | None, threads: int = 8,
                 bf16_weights: bool = False):
        config = weights.config
        self.config = config
        self._keep = []

        def keep(array):
            array = np.ascontiguousarray(array)
            if bf16_weights and array.ndim == 3 and array.shape[-1] == 34:
                n, blocks, _ = array.shape
                array = q8_dequant_bf16(array, n, blocks * 32)
            self._keep.append(array)
            return array.ctypes.data

        layers = (Layer * config.layers)()
        for index, layer in enumerate(weights.layers):
            layers[index] = Layer(keep(layer["input_norm"]), keep(layer["qkv"]),
                                  keep(layer["o"]), keep(layer["post_norm"]),
                                  keep(layer["gate_up"]), keep(layer["down"]))
        self._layers = layers
        table = None if rope is None else keep(np.asarray(rope, dtype=np.float32))
        self.struct = Stack(config.hidden, config.heads, config.kv_heads, config.head_dim,
                            config.ffn, config.layers, config.eps, table, layers,
                            keep(weights.norm), threads, int(bf16_weights))

    def forward(self, hidden, positions, cache_rows, rows_per_sequence: int,
                keys_per_sequence: int, past: int, causal: bool, k_cache, v_cache):
        """ForwardStack: returns (hidden after the layers, the final norm's
        output); k_cache / v_cache [layers][kv_heads][capacity][head_dim]
        float32 are updated in place."""
        hidden = np.array(hidden, dtype=np.float32, copy=True)
        rows = hidden.shape[0]
        output = np.zeros_like(hidden)
        positions = np.ascontiguousarray(positions, dtype=np.int32)
        cache_rows = np.ascontiguousarray(cache_rows, dtype=np.int32)
        assert k_cache.dtype == np.float32 and k_cache.flags.c_contiguous
        assert v_cache.dtype == np.float32 and v_cache.flags.c_contiguous
        capacity = k_cache.shape[2]
        lib().vo_stack_forward(ctypes.addressof(self.struct), ptr(hidden), ptr(output), rows,
                               ptr(positions), ptr(cache_rows), rows_per_sequence,
                               keys_per_sequence, past, int(causal), ptr(k_cache),
                               ptr(v_cache), capacity)
        return hidden, output


class OracleVae:
    """A vo_vae over host copies of synthetic decoder weights."""

    def __init__(self, weights):
        t = weights.tensors
        self.config = weights.config
        self._keep = []

        def keep(array):
            array = np.ascontiguousarray(array, dtype=np.float32)
            self._keep.append(array)
            return array.ctypes.data

        blocks = (VaeBlock * len(t["blocks"]))()
        for i, b in enumerate(t["blocks"]):
            units = (VaeUnit * 3)()
            for u, unit in enumerate(b["units"]):
                units[u] = VaeUnit(*(keep(unit[n]) for n in (
                    "alpha_in", "depthwise", "depthwise_bias", "alpha_out", "pointwise",
                    "pointwise_bias")))
            blocks[i] = VaeBlock(b["stride"], keep(b["scale"]), keep(b["bias"]),
                                 keep(b["alpha"]), keep(b["up"]), keep(b["up_bias"]), units)
        self._blocks = blocks
        c = self.config
        self.struct = Vae(c.latent, c.decoder_dim, len(t["blocks"]), keep(t["in_depthwise"]),
                          keep(t["in_depthwise_bias"]), keep(t["in_pointwise"]),
                          keep(t["in_pointwise_bias"]), blocks, keep(t["out_alpha"]),
                          keep(t["out_conv"]), t["out_bias"])

    def decode(self, latents: np.ndarray) -> np.ndarray:
        latents = np.ascontiguousarray(latents, dtype=np.float32)
        frames = latents.shape[0]
        out = np.zeros(frames * self.config.hop, dtype=np.float32)
        lib().vo_vae_decode(ctypes.addressof(self.struct), ptr(latents), frames, ptr(out))
        return out
