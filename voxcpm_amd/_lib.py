"""ctypes binding of libvoxcpm_amd.so, the C ABI of include/voxcpm_amd.h.

The library must have been built (voxcpm_amd.build); loading fails loudly
otherwise -- there is no fallback implementation.
"""
from __future__ import annotations

import ctypes
import pathlib

LIBRARY = pathlib.Path(__file__).resolve().parent / "libvoxcpm_amd.so"

VX_OK = 0
VX_UNSUPPORTED = 1
VX_BAD_ARG = 2
VX_HIP_ERROR = 3

# DiT evaluation paths (voxcpm_amd_internal.h).
DIT_PATH_AUTO = 0
DIT_PATH_PERSISTENT = 1
DIT_PATH_FUSED = 2
DIT_PATH_UNFUSED = 3
DIT_PATH_FUSED_REFERENCE_ORDER = 4

c_size = ctypes.c_size_t
c_int = ctypes.c_int
c_float = ctypes.c_float
c_void_p = ctypes.c_void_p


class VxError(RuntimeError):
    """A failed voxcpm_amd call: `status` is the vx_status."""

    def __init__(self, status: int, message: str):
        super().__init__(f"voxcpm_amd status {status}: {message}")
        self.status = status


class DitShape(ctypes.Structure):
    _fields_ = [(name, ctypes.c_uint32) for name in (
        "hidden", "heads", "kv_heads", "head_dim", "ffn", "layers", "patch",
        "feat", "time_in", "has_delta")] + [("eps", ctypes.c_float)]


class DitProjection(ctypes.Structure):
    _fields_ = [("weight", c_void_p), ("bias", c_void_p)]


class DitLayer(ctypes.Structure):
    _fields_ = [("input_norm", c_void_p), ("qkv", c_void_p), ("o", c_void_p),
                ("post_norm", c_void_p), ("gate_up", c_void_p),
                ("down", c_void_p)]


class DitWeights(ctypes.Structure):
    _fields_ = [("layers", ctypes.POINTER(DitLayer)), ("norm", c_void_p),
                ("rope", c_void_p), ("in_proj", DitProjection),
                ("cond_proj", DitProjection), ("out_proj", DitProjection),
                ("time_1", DitProjection), ("time_2", DitProjection),
                ("delta_1", DitProjection), ("delta_2", DitProjection),
                ("format", ctypes.c_uint32)]


VX_WEIGHTS_Q8_0 = 0
VX_WEIGHTS_BF16 = 1


class VaeUnit(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("alpha_in", "depthwise", "depthwise_bias",
                                         "alpha_out", "pointwise", "pointwise_bias")]


class VaeBlock(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("scale", "bias", "alpha", "up", "up_bias")] + [
        ("units", VaeUnit * 3)]


class VaeShape(ctypes.Structure):
    _fields_ = [("latent_dim", c_size), ("decoder_dim", c_size), ("rate_count", c_size),
                ("rates", c_size * 8)]


class VaeWeights(ctypes.Structure):
    _fields_ = [(n, c_void_p) for n in ("in_depthwise", "in_depthwise_bias", "in_pointwise",
                                         "in_pointwise_bias")] + [
        ("blocks", ctypes.POINTER(VaeBlock)), ("out_alpha", c_void_p), ("out_conv", c_void_p),
        ("out_bias", c_float)]

# GGUF components (voxcpm_amd.h).
GGUF_MODEL = 0
GGUF_VAE = 1

# Stack paths (voxcpm_amd_internal.h).
STACK_PATH_AUTO = 0
STACK_PATH_FUSED = 2
STACK_PATH_UNFUSED = 3
STACK_PATH_ROWS = 4


class StackShape(ctypes.Structure):
    _fields_ = [(name, c_size) for name in (
        "hidden", "heads", "kv_heads", "head_dim", "ffn", "layers")] + [
        ("eps", ctypes.c_float), ("rope", c_int)]


class StackWeights(ctypes.Structure):
    _fields_ = [("layers", ctypes.POINTER(DitLayer)), ("norm", c_void_p),
                ("rope", c_void_p), ("format", ctypes.c_uint32)]


_SIGNATURES = {
    "vx_last_error": ([], ctypes.c_char_p),
    "vx_last_hip_error": ([], c_int),
    "vx_version": ([], ctypes.c_char_p),
    "vx_q8_packed_bytes": ([c_size, c_size], c_size),
    "vx_q8_pack": ([c_void_p, c_size, c_size, c_void_p, c_void_p], c_int),
    "vx_q8_unpack_blocks": ([c_void_p, c_size, c_size, c_void_p, c_void_p], c_int),
    "vx_q8_unpack_bf16": ([c_void_p, c_size, c_size, c_void_p, c_void_p], c_int),
    "vx_scratch_create": ([ctypes.POINTER(c_void_p), c_size, c_size], c_int),
    "vx_scratch_destroy": ([c_void_p], None),
    "vx_q8_linear": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                      c_int, c_void_p, c_void_p], c_int),
    "vx_q8_linear_noalloc": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                              c_int, c_void_p], c_int),
    "vx_q8_linear_bf16": ([c_void_p, c_void_p, c_void_p, c_size, c_size,
                           c_size, c_void_p, c_void_p], c_int),
    "vx_q8_linear_planned": ([c_void_p, c_void_p, c_void_p, c_size, c_size,
                              c_size, c_int, c_void_p, c_int, c_int, c_int,
                              c_void_p], c_int),
    "vx_q8_linear_engine": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                             c_int, c_int, c_int, c_int, c_void_p], c_int),
    "vx_q8_linear_gemm": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                           c_int, c_int, c_void_p, c_void_p], c_int),
    "vx_bf16_linear_gemm": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                             c_int, c_int, c_void_p, c_void_p], c_int),
    "vx_q8_plan": ([c_size, c_size, c_size, c_void_p, c_void_p], c_int),
    "vx_q8_prefill_plan": ([c_size, c_size, c_size, c_void_p, c_void_p], c_int),
    "vx_bf16_packed_bytes": ([c_size, c_size], c_size),
    "vx_bf16_pack": ([c_void_p, c_size, c_size, c_void_p, c_void_p], c_int),
    "vx_bf16_unpack": ([c_void_p, c_size, c_size, c_void_p, c_void_p], c_int),
    "vx_bf16_linear": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                        c_int, c_void_p, c_void_p], c_int),
    "vx_bf16_linear_rows": ([c_void_p, c_void_p, c_void_p, c_size, c_size, c_size,
                             c_int, c_void_p], c_int),
    "vx_test_pack_bf16": ([c_void_p, c_void_p, c_size, c_void_p], c_int),
    "vx_stream_read": ([c_void_p, c_size, ctypes.c_uint32, c_void_p, c_void_p], c_int),
    "vx_handoff": ([c_void_p, c_void_p, c_size, c_int, c_int, ctypes.c_uint32, c_void_p,
                    c_void_p], c_int),
    "vx_rms_norm": ([c_void_p, c_void_p, c_void_p, c_void_p, c_size, c_size,
                     c_float, c_void_p], c_int),
    "vx_qkv_rope": ([c_void_p] * 7 + [c_size] * 5 + [c_void_p], c_int),
    "vx_attention": ([c_void_p] * 4 + [c_size] * 4 + [c_int] + [c_size] * 4
                     + [c_void_p], c_int),
    "vx_swiglu": ([c_void_p, c_void_p, c_size, c_size, c_void_p], c_int),
    "vx_add_bias": ([c_void_p, c_void_p, c_size, c_size, c_void_p], c_int),
    "vx_to_bf16": ([c_void_p, c_void_p, c_size, c_int, c_void_p], c_int),
    "vx_gather_rows": ([c_void_p, c_void_p, c_void_p, c_size, c_size,
                        c_void_p], c_int),
    "vx_assemble_dit": ([c_void_p] * 5 + [c_size, c_size, c_void_p], c_int),
    "vx_guided_euler": ([c_void_p, c_void_p, c_size, c_float, c_float, c_int,
                         c_void_p], c_int),
    "vx_dit_create": ([ctypes.POINTER(c_void_p), ctypes.POINTER(DitShape),
                       ctypes.POINTER(DitWeights)], c_int),
    "vx_dit_destroy": ([c_void_p], None),
    "vx_dit_time_vector": ([c_void_p, c_float, c_void_p, c_void_p], c_int),
    "vx_dit_cond_rows": ([c_void_p, c_void_p, c_void_p, c_void_p], c_int),
    "vx_dit_eval": ([c_void_p] * 6 + [c_void_p], c_int),
    "vx_dit_velocity": ([c_void_p] * 4 + [c_float, c_void_p, c_void_p], c_int),
    "vx_dit_patch": ([c_void_p] * 7 + [c_size, c_float, c_int, c_void_p], c_int),
    "vx_dit_status": ([c_void_p], c_int),
    "vx_dit_set_path": ([c_void_p, c_int], c_int),
    "vx_dit_path": ([c_void_p], c_int),
    "vx_dit_set_trace": ([c_void_p, c_void_p, c_size], c_int),
    "vx_dit_trace_bytes": ([c_void_p], c_size),
    "vx_stack_create": ([ctypes.POINTER(c_void_p), ctypes.POINTER(StackShape),
                         ctypes.POINTER(StackWeights)], c_int),
    "vx_stack_destroy": ([c_void_p], None),
    # (stack, hidden, output, rows, positions, cache_rows, rows_per_sequence,
    #  keys_per_sequence, past, causal, k_cache, v_cache, capacity, stream)
    "vx_stack_forward": ([c_void_p, c_void_p, c_void_p, c_size, c_void_p, c_void_p,
                          c_size, c_size, c_size, c_int, c_void_p, c_void_p, c_size,
                          c_void_p], c_int),
    "vx_stack_set_path": ([c_void_p, c_int], c_int),
    "vx_stack_path": ([c_void_p, c_size], c_int),
    "vx_split_attention": ([c_void_p] * 4 + [c_size] * 4 + [c_int] + [c_size] * 4
                           + [c_void_p, c_size, c_void_p], c_int),
    "vx_split_attention_floats": ([c_size] * 5, c_size),
    "vx_gguf_open": ([ctypes.c_char_p, c_int, ctypes.POINTER(c_void_p)], c_int),
    "vx_gguf_close": ([c_void_p], None),
    "vx_gguf_last_error": ([], ctypes.c_char_p),
    "vx_gguf_tensor_count": ([c_void_p, c_int], c_size),
    "vx_gguf_tensor": ([c_void_p, c_int, c_size, ctypes.POINTER(ctypes.c_char_p),
                        ctypes.POINTER(ctypes.c_uint32), ctypes.POINTER(c_size),
                        ctypes.POINTER(c_size), ctypes.POINTER(c_void_p),
                        ctypes.POINTER(ctypes.c_uint64)], c_int),
    "vx_gguf_find": ([c_void_p, c_int, ctypes.c_char_p, ctypes.POINTER(c_size)], c_int),
    "vx_gguf_embedded": ([c_void_p, ctypes.c_char_p, ctypes.POINTER(c_size)], c_void_p),
    "vx_gguf_upload_q8": ([c_void_p, c_int, c_size, c_void_p, c_size, c_void_p], c_int),
    "vx_vae_create": ([ctypes.POINTER(c_void_p), ctypes.POINTER(VaeShape),
                       ctypes.POINTER(VaeWeights)], c_int),
    "vx_vae_destroy": ([c_void_p], None),
    "vx_vae_reset": ([c_void_p, c_void_p], c_int),
    "vx_vae_hop": ([c_void_p], c_size),
    "vx_vae_max_frames": ([c_void_p], c_size),
    "vx_vae_decode": ([c_void_p, c_void_p, c_size, c_void_p, c_void_p], c_int),
    "vx_euler_schedule": ([c_size, c_float, c_int, c_void_p, c_void_p,
                           c_void_p], c_int),
    "vx_rope_table": ([ctypes.c_double, c_size, c_void_p, c_float, c_size,
                       c_void_p], c_int),
}

_lib: ctypes.CDLL | None = None


def lib() -> ctypes.CDLL:
    """The loaded library (raises if it has not been built)."""
    global _lib
    if _lib is None:
        if not LIBRARY.exists():
            raise RuntimeError(
                f"{LIBRARY} is missing: build it with `python -m voxcpm_amd.build`"
                " (there is no fallback path)")
        handle = ctypes.CDLL(str(LIBRARY))
        for name, (args, result) in _SIGNATURES.items():
            function = getattr(handle, name)
            function.argtypes = args
            function.restype = result
        _lib = handle
    return _lib


def check(status: int) -> None:
    """Raises VxError for a failed status."""
    if status != VX_OK:
        raise VxError(status, lib().vx_last_error().decode())
