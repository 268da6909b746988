"""Python entry points over the C ABI, with torch tensors as device memory.

Every function calls libvoxcpm_amd.so; torch only allocates device memory
and supplies the stream. bf16 tensors are torch.bfloat16 (the same bits as
the ABI's uint16 bfloat16).
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import synth
from ._lib import (VX_WEIGHTS_BF16, VX_WEIGHTS_Q8_0, DitLayer, DitProjection, DitShape,
                   DitWeights, StackShape, StackWeights, VaeBlock, VaeShape, VaeUnit,
                   VaeWeights, check, lib)

__all__ = [
    "Scratch", "Dit", "q8_pack", "q8_unpack_blocks", "q8_unpack_bf16",
    "q8_linear", "q8_linear_bf16", "q8_plan", "bf16_pack", "bf16_unpack", "bf16_linear",
    "bf16_linear_rows", "stream_read", "handoff", "euler_schedule", "rope_table", "Stack",
    "split_attention", "Gguf", "Vae",
]


def _ptr(tensor: torch.Tensor | None) -> ctypes.c_void_p | None:
    return None if tensor is None else ctypes.c_void_p(tensor.data_ptr())


def _stream(stream: torch.cuda.Stream | None) -> ctypes.c_void_p:
    stream = stream or torch.cuda.current_stream()
    return ctypes.c_void_p(stream.cuda_stream)


def _device(device) -> torch.device:
    return torch.device(device if device is not None else "cuda")


# ---- Q8_0 panels -----------------------------------------------------------

def q8_pack(blocks: torch.Tensor, n: int, k: int, stream=None) -> torch.Tensor:
    """GGML Q8_0 blocks (uint8 [n][k/32][34] on the device) -> panels."""
    packed = torch.empty(lib().vx_q8_packed_bytes(n, k), dtype=torch.uint8,
                         device=blocks.device)
    check(lib().vx_q8_pack(_ptr(blocks), n, k, _ptr(packed), _stream(stream)))
    return packed


def q8_unpack_blocks(packed: torch.Tensor, n: int, k: int,
                     stream=None) -> torch.Tensor:
    blocks = torch.empty((n, k // 32, 34), dtype=torch.uint8,
                         device=packed.device)
    check(lib().vx_q8_unpack_blocks(_ptr(packed), n, k, _ptr(blocks),
                                    _stream(stream)))
    return blocks


def q8_unpack_bf16(packed: torch.Tensor, n: int, k: int,
                   stream=None) -> torch.Tensor:
    out = torch.empty((n, k), dtype=torch.bfloat16, device=packed.device)
    check(lib().vx_q8_unpack_bf16(_ptr(packed), n, k, _ptr(out),
                                  _stream(stream)))
    return out


class Scratch:
    """vx_scratch: split-reduction scratch of the products."""

    def __init__(self, max_m: int, max_n: int):
        handle = ctypes.c_void_p()
        check(lib().vx_scratch_create(ctypes.byref(handle), max_m, max_n))
        self.handle = handle

    def close(self) -> None:
        if self.handle:
            lib().vx_scratch_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def q8_linear(x: torch.Tensor, packed: torch.Tensor, n: int,
              y: torch.Tensor | None = None, accumulate: bool = False,
              scratch: Scratch | None = None, plan: tuple | None = None,
              stream=None) -> torch.Tensor:
    """y[m][n] (+)= x[m][k] W^T; x bf16 [m][k], y float32 [m][n].

    `plan` = (row_groups, waves, splits) forces the split (m <= 128)."""
    m, k = x.shape
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    handle = scratch.handle if scratch is not None else None
    if plan is None:
        status = lib().vx_q8_linear(_ptr(x), _ptr(packed), _ptr(y), m, k, n,
                                    int(accumulate), handle, _stream(stream))
    else:
        status = lib().vx_q8_linear_planned(
            _ptr(x), _ptr(packed), _ptr(y), m, k, n, int(accumulate), handle,
            plan[0], plan[1], plan[2], _stream(stream))
    check(status)
    return y


def q8_linear_bf16(x: torch.Tensor, packed: torch.Tensor, n: int,
                   y: torch.Tensor | None = None,
                   scratch: Scratch | None = None, stream=None) -> torch.Tensor:
    m, k = x.shape
    if y is None:
        y = torch.empty((m, n), dtype=torch.bfloat16, device=x.device)
    handle = scratch.handle if scratch is not None else None
    check(lib().vx_q8_linear_bf16(_ptr(x), _ptr(packed), _ptr(y), m, k, n,
                                  handle, _stream(stream)))
    return y


# ---- bf16 weights -----------------------------------------------------------

def bf16_pack(rows: torch.Tensor, stream=None) -> torch.Tensor:
    """bf16 weight rows [n][k] (on the device) -> panels."""
    n, k = rows.shape
    packed = torch.empty(lib().vx_bf16_packed_bytes(n, k), dtype=torch.uint8,
                         device=rows.device)
    check(lib().vx_bf16_pack(_ptr(rows), n, k, _ptr(packed), _stream(stream)))
    return packed


def bf16_unpack(packed: torch.Tensor, n: int, k: int, stream=None) -> torch.Tensor:
    rows = torch.empty((n, k), dtype=torch.bfloat16, device=packed.device)
    check(lib().vx_bf16_unpack(_ptr(packed), n, k, _ptr(rows), _stream(stream)))
    return rows


def bf16_linear(x: torch.Tensor, packed: torch.Tensor, n: int,
                y: torch.Tensor | None = None, accumulate: bool = False,
                scratch: Scratch | None = None, stream=None) -> torch.Tensor:
    """y[m][n] (+)= x[m][k] W^T on bf16 panels; x bf16 [m][k], y float32."""
    m, k = x.shape
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    handle = scratch.handle if scratch is not None else None
    check(lib().vx_bf16_linear(_ptr(x), _ptr(packed), _ptr(y), m, k, n,
                               int(accumulate), handle, _stream(stream)))
    return y


def bf16_linear_rows(x: torch.Tensor, w: torch.Tensor, y: torch.Tensor | None = None,
                     accumulate: bool = False, stream=None) -> torch.Tensor:
    """y[m][n] (+)= x[m][k] W^T on bf16 rows W [n][k], m <= 32."""
    m, k = x.shape
    n = w.shape[0]
    if y is None:
        y = torch.empty((m, n), dtype=torch.float32, device=x.device)
    check(lib().vx_bf16_linear_rows(_ptr(x), _ptr(w), _ptr(y), m, k, n,
                                    int(accumulate), _stream(stream)))
    return y


def stream_read(data: torch.Tensor, sink: torch.Tensor, never: int = 0x9E3779B9,
                stream=None) -> None:
    """One coalesced read of `data`'s bytes (the per-launch read ceiling);
    `sink` (int32 [1]) changes only if the bytes' XOR equals `never`."""
    check(lib().vx_stream_read(_ptr(data), data.numel() * data.element_size(), never,
                               _ptr(sink), _stream(stream)))


def handoff(data_in: torch.Tensor | None, data_out: torch.Tensor | None, nbytes: int,
            workgroups: int, threads: int, sink: torch.Tensor, never: int = 0x9E3779B9,
            stream=None) -> None:
    """One launch of the hand-off probe (vx_handoff): every workgroup reads
    `nbytes` of data_in, together they write data_out = data_in + 1; with
    nbytes = 0 an empty launch of that grid."""
    check(lib().vx_handoff(_ptr(data_in) if data_in is not None else None,
                           _ptr(data_out) if data_out is not None else None, nbytes,
                           workgroups, threads, never, _ptr(sink), _stream(stream)))


def q8_plan(m: int, k: int, n: int, scratch: Scratch | None = None) -> dict:
    out = (ctypes.c_int32 * 7)()
    check(lib().vx_q8_plan(m, k, n, scratch.handle if scratch else None, out))
    names = ("mt", "rg", "waves", "tiles", "splits", "pairs_per_split",
             "pairs_per_wave")
    return dict(zip(names, list(out)))


# ---- host-side schedule and tables -----------------------------------------

def euler_schedule(timesteps: int, sway: float = 1.0, skip: bool = True):
    """(t, dt, evaluate) numpy arrays of EulerSchedule."""
    t = np.zeros(timesteps, dtype=np.float32)
    dt = np.zeros(timesteps, dtype=np.float32)
    evaluate = np.zeros(timesteps, dtype=np.int32)
    check(lib().vx_euler_schedule(timesteps, sway, int(skip),
                                  t.ctypes.data, dt.ctypes.data,
                                  evaluate.ctypes.data))
    return t, dt, evaluate


def rope_table(theta: float, dim: int, factors, scaling: float,
               positions: int) -> np.ndarray:
    table = np.zeros((positions, dim), dtype=np.float32)
    f = None
    if factors is not None:
        f = np.ascontiguousarray(factors, dtype=np.float64)
    check(lib().vx_rope_table(theta, dim, None if f is None else f.ctypes.data,
                              scaling, positions, table.ctypes.data))
    return table


# ---- the DiT -----------------------------------------------------------------

class Dit:
    """vx_dit over device copies of synthetic (or given) host weights."""

    def __init__(self, weights: synth.DitWeightsHost, device=None,
                 stream=None, bf16_weights: bool = False):
        """`bf16_weights`: every matrix as bf16 panels of bf16(scale q), the
        bf16 expansion of its Q8_0 blocks (the DiT on bf16 weights)."""
        self.config = config = weights.config
        device = _device(device)
        self._keep = []

        def upload_q8(blocks: np.ndarray) -> torch.Tensor:
            n, kb, _ = blocks.shape
            raw = torch.from_numpy(np.ascontiguousarray(blocks)).to(device)
            packed = q8_pack(raw, n, kb * 32, stream)
            if bf16_weights:
                packed = bf16_pack(q8_unpack_bf16(packed, n, kb * 32, stream), stream)
            self._keep.append(packed)
            return packed

        def upload_bf16(bits: np.ndarray) -> torch.Tensor:
            tensor = torch.from_numpy(bits.view(np.int16).copy()).to(device)
            self._keep.append(tensor)
            return tensor

        layer_array = (DitLayer * config.layers)()
        for index, layer in enumerate(weights.layers):
            layer_array[index] = DitLayer(
                upload_bf16(layer["input_norm"]).data_ptr(),
                upload_q8(layer["qkv"]).data_ptr(),
                upload_q8(layer["o"]).data_ptr(),
                upload_bf16(layer["post_norm"]).data_ptr(),
                upload_q8(layer["gate_up"]).data_ptr(),
                upload_q8(layer["down"]).data_ptr())
        projections = {}
        for name in synth.PROJECTIONS:
            if name in weights.projections:
                blocks, bias = weights.projections[name]
                projections[name] = DitProjection(
                    upload_q8(blocks).data_ptr(), upload_bf16(bias).data_ptr())
            else:
                projections[name] = DitProjection(None, None)
        rope_ptr = None
        if weights.rope is not None:
            rope = torch.from_numpy(np.ascontiguousarray(
                weights.rope, dtype=np.float32)).to(device)
            self._keep.append(rope)
            rope_ptr = rope.data_ptr()
        self._layers = layer_array
        self._weights = DitWeights(
            layer_array, upload_bf16(weights.norm).data_ptr(), rope_ptr,
            **projections, format=VX_WEIGHTS_BF16 if bf16_weights else VX_WEIGHTS_Q8_0)
        self._shape = DitShape(
            config.hidden, config.heads, config.kv_heads, config.head_dim,
            config.ffn, config.layers, config.patch, config.feat,
            config.time_in, int(config.has_delta), config.eps)
        torch.cuda.synchronize(device)
        handle = ctypes.c_void_p()
        check(lib().vx_dit_create(ctypes.byref(handle),
                                  ctypes.byref(self._shape),
                                  ctypes.byref(self._weights)))
        self.handle = handle
        self.device = device

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().vx_dit_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def set_path(self, path: int) -> None:
        """Selects the evaluation path (voxcpm_amd._lib.DIT_PATH_*)."""
        check(lib().vx_dit_set_path(self.handle, path))

    @property
    def path(self) -> int:
        """The evaluation path that runs (AUTO resolved)."""
        return lib().vx_dit_path(self.handle)

    def set_trace(self, enable: bool = True) -> torch.Tensor | None:
        """Records persistent evaluations' timestamps into a new int64 device
        tensor [grid][barriers + 1][4] (returned), or stops recording."""
        if not enable:
            check(lib().vx_dit_set_trace(self.handle, None, 0))
            self._trace = None
            return None
        words = lib().vx_dit_trace_bytes(self.handle) // 8
        self._trace = torch.zeros(words, dtype=torch.int64, device=self.device)
        check(lib().vx_dit_set_trace(self.handle, _ptr(self._trace), words * 8))
        return self._trace

    def status(self) -> None:
        """Synchronizes; raises VxError if a persistent evaluation timed out."""
        check(lib().vx_dit_status(self.handle))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def _f32(self, *shape) -> torch.Tensor:
        return torch.empty(shape, dtype=torch.float32, device=self.device)

    def time_vector(self, t: float, stream=None) -> torch.Tensor:
        out = self._f32(self.config.hidden)
        check(lib().vx_dit_time_vector(self.handle, t, _ptr(out),
                                       _stream(stream)))
        return out

    def cond_rows(self, cond_latent: torch.Tensor, stream=None) -> torch.Tensor:
        out = self._f32(self.config.patch, self.config.hidden)
        check(lib().vx_dit_cond_rows(self.handle, _ptr(cond_latent), _ptr(out),
                                     _stream(stream)))
        return out

    def eval(self, mu, cond_rows, x, time_vector, stream=None) -> torch.Tensor:
        out = self._f32(2, self.config.patch, self.config.feat)
        check(lib().vx_dit_eval(self.handle, _ptr(mu), _ptr(cond_rows), _ptr(x),
                                _ptr(time_vector), _ptr(out), _stream(stream)))
        return out

    def velocity(self, mu, cond_latent, x, t: float, stream=None) -> torch.Tensor:
        out = self._f32(2, self.config.patch, self.config.feat)
        check(lib().vx_dit_velocity(self.handle, _ptr(mu), _ptr(cond_latent),
                                    _ptr(x), t, _ptr(out), _stream(stream)))
        return out

    def patch(self, mu, cond_latent, x, t, dt, evaluate, cfg: float,
              zero_star: bool, stream=None) -> torch.Tensor:
        """Runs the sampler in place on x; returns x."""
        t = np.ascontiguousarray(t, dtype=np.float32)
        dt = np.ascontiguousarray(dt, dtype=np.float32)
        evaluate = np.ascontiguousarray(evaluate, dtype=np.int32)
        check(lib().vx_dit_patch(
            self.handle, _ptr(mu), _ptr(cond_latent), _ptr(x), t.ctypes.data,
            dt.ctypes.data, evaluate.ctypes.data, len(t), cfg, int(zero_star),
            _stream(stream)))
        return x


def split_attention(q: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor,
                    rows_per_sequence: int, keys_per_sequence: int, past: int,
                    causal: bool, heads: int, kv_heads: int, stream=None) -> torch.Tensor:
    """The stack's attention on one layer's cache: q float32 [rows][heads][D],
    k_cache / v_cache float32 [kv_heads][capacity][D] -> bf16 [rows][heads][D]."""
    rows, _, head_dim = q.shape
    capacity = k_cache.shape[1]
    out = torch.empty((rows, heads, head_dim), dtype=torch.bfloat16, device=q.device)
    floats = lib().vx_split_attention_floats(rows, heads, head_dim, past, rows_per_sequence)
    partials = torch.empty(max(floats, 1), dtype=torch.float32, device=q.device)
    check(lib().vx_split_attention(_ptr(q), _ptr(k_cache), _ptr(v_cache), _ptr(out), rows,
                                   rows_per_sequence, keys_per_sequence, past, int(causal),
                                   heads, kv_heads, head_dim, capacity,
                                   _ptr(partials) if floats else None, floats,
                                   _stream(stream)))
    return out


class Stack:
    """vx_stack (ForwardStack with a key/value cache) over device copies of
    synthetic stack weights (synth.StackWeightsHost, or the same fields
    holding device tensors: uint8 Q8_0 blocks, int16 bf16 bits)."""

    def __init__(self, weights: synth.StackWeightsHost, rope: np.ndarray | None,
                 device=None, stream=None, bf16_weights: bool = False):
        self.config = config = weights.config
        device = _device(device)
        self._keep = []

        def upload_q8(blocks) -> torch.Tensor:
            # GGML Q8_0 blocks [n][k / 32][34]: host numpy or device uint8.
            n, kb, _ = blocks.shape
            raw = blocks.to(device) if isinstance(blocks, torch.Tensor) else \
                torch.from_numpy(np.ascontiguousarray(blocks)).to(device)
            packed = q8_pack(raw, n, kb * 32, stream)
            if bf16_weights:
                packed = bf16_pack(q8_unpack_bf16(packed, n, kb * 32, stream), stream)
            self._keep.append(packed)
            return packed

        def upload_bf16(bits) -> torch.Tensor:
            tensor = bits.to(device) if isinstance(bits, torch.Tensor) else \
                torch.from_numpy(bits.view(np.int16).copy()).to(device)
            self._keep.append(tensor)
            return tensor

        layer_array = (DitLayer * config.layers)()
        for index, layer in enumerate(weights.layers):
            layer_array[index] = DitLayer(
                upload_bf16(layer["input_norm"]).data_ptr(),
                upload_q8(layer["qkv"]).data_ptr(),
                upload_q8(layer["o"]).data_ptr(),
                upload_bf16(layer["post_norm"]).data_ptr(),
                upload_q8(layer["gate_up"]).data_ptr(),
                upload_q8(layer["down"]).data_ptr())
        rope_ptr = None
        if config.rope:
            table = torch.from_numpy(np.ascontiguousarray(rope, dtype=np.float32)).to(device)
            self._keep.append(table)
            rope_ptr = table.data_ptr()
        self._layers = layer_array
        self._weights = StackWeights(layer_array, upload_bf16(weights.norm).data_ptr(),
                                     rope_ptr,
                                     VX_WEIGHTS_BF16 if bf16_weights else VX_WEIGHTS_Q8_0)
        self._shape = StackShape(config.hidden, config.heads, config.kv_heads,
                                 config.head_dim, config.ffn, config.layers, config.eps,
                                 int(config.rope))
        torch.cuda.synchronize(device)
        handle = ctypes.c_void_p()
        check(lib().vx_stack_create(ctypes.byref(handle), ctypes.byref(self._shape),
                                    ctypes.byref(self._weights)))
        self.handle = handle
        self.device = device

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().vx_stack_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        self.close()

    def set_path(self, path: int) -> None:
        """Selects the path (voxcpm_amd._lib.STACK_PATH_*)."""
        check(lib().vx_stack_set_path(self.handle, path))

    def path(self, rows: int) -> int:
        return lib().vx_stack_path(self.handle, rows)

    def cache(self, capacity: int) -> tuple[torch.Tensor, torch.Tensor]:
        """A zeroed key/value cache [layers][kv_heads][capacity][head_dim]."""
        c = self.config
        shape = (c.layers, c.kv_heads, capacity, c.head_dim)
        return (torch.zeros(shape, dtype=torch.float32, device=self.device),
                torch.zeros(shape, dtype=torch.float32, device=self.device))

    def forward(self, hidden: torch.Tensor, output: torch.Tensor, positions: torch.Tensor,
                cache_rows: torch.Tensor, rows_per_sequence: int, keys_per_sequence: int,
                past: int, causal: bool, k_cache: torch.Tensor, v_cache: torch.Tensor,
                stream=None) -> None:
        """ForwardStack: hidden float32 [rows][hidden] (in place), output
        float32 [rows][hidden], positions / cache_rows int32 [rows]."""
        rows = hidden.shape[0]
        check(lib().vx_stack_forward(self.handle, _ptr(hidden), _ptr(output), rows,
                                     _ptr(positions), _ptr(cache_rows), rows_per_sequence,
                                     keys_per_sequence, past, int(causal), _ptr(k_cache),
                                     _ptr(v_cache), k_cache.shape[2], _stream(stream)))


class Gguf:
    """vx_gguf: a GGUF file mapped read-only -- the audio.cpp VoxCPM2 layout
    (`voxcpm2=True`, ModelFiles::Open's GGUF branch) or any GGUF with its
    own tensor names."""

    def __init__(self, path: str, voxcpm2: bool = True):
        from ._lib import VxError
        handle = ctypes.c_void_p()
        status = lib().vx_gguf_open(str(path).encode(), int(voxcpm2), ctypes.byref(handle))
        if status != 0:
            raise VxError(status, lib().vx_gguf_last_error().decode())
        self.handle = handle

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().vx_gguf_close(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        self.close()

    def tensors(self, component: int = 0) -> list[dict]:
        """Name, GGML type, shape (outermost first) and bytes (a numpy copy)
        of every tensor of a component (voxcpm_amd._lib.GGUF_MODEL / _VAE)."""
        out = []
        for index in range(lib().vx_gguf_tensor_count(self.handle, component)):
            name = ctypes.c_char_p()
            kind = ctypes.c_uint32()
            shape = (ctypes.c_size_t * 8)()
            rank = ctypes.c_size_t()
            data = ctypes.c_void_p()
            size = ctypes.c_uint64()
            check(lib().vx_gguf_tensor(self.handle, component, index, ctypes.byref(name),
                                       ctypes.byref(kind), shape, ctypes.byref(rank),
                                       ctypes.byref(data), ctypes.byref(size)))
            raw = np.ctypeslib.as_array(ctypes.cast(data, ctypes.POINTER(ctypes.c_uint8)),
                                        shape=(size.value,)).copy()
            out.append({"name": name.value.decode(), "type": kind.value,
                        "shape": tuple(shape[d] for d in range(rank.value)), "bytes": raw})
        return out

    def embedded(self, file: str) -> str | None:
        size = ctypes.c_size_t()
        text = lib().vx_gguf_embedded(self.handle, file.encode(), ctypes.byref(size))
        return None if text is None else ctypes.string_at(text, size.value).decode()

    def upload_q8(self, name: str, component: int = 0, device=None,
                  stream=None) -> torch.Tensor:
        """A Q8_0 matrix [out][in] of the file as Q8_0 panels on the device."""
        from ._lib import VxError
        index = ctypes.c_size_t()
        status = lib().vx_gguf_find(self.handle, component, name.encode(), ctypes.byref(index))
        if status != 0:
            raise VxError(status, lib().vx_gguf_last_error().decode())
        shape = (ctypes.c_size_t * 8)()
        rank = ctypes.c_size_t()
        check(lib().vx_gguf_tensor(self.handle, component, index.value, None, None, shape,
                                   ctypes.byref(rank), None, None))
        out, inner = (shape[0], shape[1]) if rank.value == 2 else (1, 32)
        packed = torch.empty(lib().vx_q8_packed_bytes(out, inner), dtype=torch.uint8,
                             device=_device(device))
        status = lib().vx_gguf_upload_q8(self.handle, component, index.value, _ptr(packed),
                                         packed.numel(), _stream(stream))
        if status != 0:
            raise VxError(status, lib().vx_gguf_last_error().decode())
        return packed


class Vae:
    """vx_vae (AudioVAE V2's streaming decoder) over device copies of
    float32 decoder weights (synth.VaeWeightsHost; numpy arrays or device
    tensors)."""

    def __init__(self, weights, device=None, stream=None):
        self.config = config = weights.config
        t = weights.tensors
        device = _device(device)
        self._keep = []

        def up(array) -> int:
            tensor = array.to(device, torch.float32).contiguous() \
                if isinstance(array, torch.Tensor) else \
                torch.from_numpy(np.ascontiguousarray(array, dtype=np.float32)).to(device)
            self._keep.append(tensor)
            return tensor.data_ptr()

        blocks = (VaeBlock * len(t["blocks"]))()
        for i, b in enumerate(t["blocks"]):
            units = (VaeUnit * 3)()
            for u, unit in enumerate(b["units"]):
                units[u] = VaeUnit(*(up(unit[n]) for n in (
                    "alpha_in", "depthwise", "depthwise_bias", "alpha_out", "pointwise",
                    "pointwise_bias")))
            blocks[i] = VaeBlock(up(b["scale"]), up(b["bias"]), up(b["alpha"]), up(b["up"]),
                                 up(b["up_bias"]), units)
        self._blocks = blocks
        rates = (ctypes.c_size_t * 8)(*config.rates)
        self._shape = VaeShape(config.latent, config.decoder_dim, len(config.rates), rates)
        self._weights = VaeWeights(up(t["in_depthwise"]), up(t["in_depthwise_bias"]),
                                   up(t["in_pointwise"]), up(t["in_pointwise_bias"]), blocks,
                                   up(t["out_alpha"]), up(t["out_conv"]), t["out_bias"])
        torch.cuda.synchronize(device)
        handle = ctypes.c_void_p()
        check(lib().vx_vae_create(ctypes.byref(handle), ctypes.byref(self._shape),
                                  ctypes.byref(self._weights)))
        self.handle = handle
        self.device = device
        self.hop = lib().vx_vae_hop(handle)
        self.max_frames = lib().vx_vae_max_frames(handle)

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().vx_vae_destroy(self.handle)
            self.handle = ctypes.c_void_p()

    def __del__(self):
        self.close()

    def reset(self, stream=None) -> None:
        check(lib().vx_vae_reset(self.handle, _stream(stream)))

    def decode(self, latents: torch.Tensor, samples: torch.Tensor | None = None,
               stream=None) -> torch.Tensor:
        """latents float32 [frames][latent] on the device -> samples
        [frames * hop], continuing the stream."""
        # The C ABI takes bare pointers and a frame count: the tensors must
        # be exactly what it reads and writes.
        if latents.dtype != torch.float32 or latents.dim() != 2 or not latents.is_contiguous():
            raise ValueError("latents must be a contiguous float32 [frames][latent] tensor")
        if latents.shape[1] != self.config.latent:
            raise ValueError(f"latents have {latents.shape[1]} channels, the decoder "
                             f"takes {self.config.latent}")
        if latents.device.type != "cuda" or (self.device.index is not None and
                                              latents.device.index != self.device.index):
            raise ValueError(f"latents are on {latents.device}, the decoder on {self.device}")
        frames = latents.shape[0]
        if samples is None:
            samples = torch.empty(frames * self.hop, dtype=torch.float32, device=latents.device)
        elif (samples.dtype != torch.float32 or not samples.is_contiguous() or
              samples.numel() < frames * self.hop or samples.device != latents.device):
            raise ValueError(f"samples must be a contiguous float32 tensor of at least "
                             f"{frames * self.hop} values on {latents.device}")
        check(lib().vx_vae_decode(self.handle, _ptr(latents), frames, _ptr(samples),
                                  _stream(stream)))
        return samples
