"""The GGUF reader (voxcpm_amd/host/gguf.cpp) on files written from the
published format by tests/gguf_file.py: every metadata type, tensors of
each type the VoxCPM2 GGUFs hold at several ranks and alignments, the
audio.cpp VoxCPM2 layout the reference opens (model_files.cpp:111-184:
component prefixes, abbreviated names, embedded config and tokenizer), and
malformed files, which fail without a crash. No GPU: parsing only."""
import numpy as np
import pytest

import gguf_file as gf
from voxcpm_amd import _lib, synth


@pytest.fixture(scope="module")
def ops():
    from voxcpm_amd import ops
    _lib.lib()
    return ops


def q8_tensor(rng, out, inner):
    blocks = synth.q8_blocks(rng, out, inner)
    return np.ascontiguousarray(blocks).tobytes()


def test_raw_gguf_metadata_and_tensors(ops, tmp_path):
    rng = synth.Rng(61, 1)
    f32 = rng.normal(6 * 5).astype(np.float32)
    f16 = rng.normal(64).astype(np.float16)
    bf16 = synth.bf16_bits(rng.normal(3 * 2 * 8).astype(np.float32))
    i32 = np.arange(7, dtype=np.int32) - 3
    q8 = q8_tensor(rng, 3, 64)
    tensors = [("a.f32", gf.GGML_F32, [5, 6], f32.tobytes()),
               ("b.f16", gf.GGML_F16, [64], f16.tobytes()),
               ("c.bf16", gf.GGML_BF16, [8, 2, 3], bf16.tobytes()),
               ("d.i32", gf.GGML_I32, [7], i32.tobytes()),
               ("e.q8", gf.GGML_Q8_0, [64, 3], q8)]
    metadata = [("k.u8", gf.U8, 200), ("k.i8", gf.I8, -5), ("k.u16", gf.U16, 60000),
                ("k.i16", gf.I16, -30000), ("k.u32", gf.U32, 4000000000),
                ("k.i32", gf.I32, -7), ("k.f32", gf.F32, 1.5), ("k.bool", gf.BOOL, True),
                ("k.str", gf.STRING, "text"), ("k.u64", gf.U64, 2 ** 63 + 5),
                ("k.i64", gf.I64, -(2 ** 40)), ("k.f64", gf.F64, 2.25),
                ("k.arr", gf.ARRAY, (gf.STRING, ["x", "yz"])),
                ("k.ints", gf.ARRAY, (gf.I16, [1, -2, 3]))]
    for alignment in (32, 64):
        path = tmp_path / f"raw{alignment}.gguf"
        meta = metadata + ([("general.alignment", gf.U32, alignment)] if alignment != 32 else [])
        gf.write(path, meta, tensors, alignment=alignment)
        got = ops.Gguf(path, voxcpm2=False).tensors()
        assert [t["name"] for t in got] == [t[0] for t in tensors]
        for t, (name, kind, dims, data) in zip(got, tensors):
            assert t["type"] == kind
            assert t["shape"] == tuple(reversed(dims)), name  # outermost first
            assert t["bytes"].tobytes() == data, name


def voxcpm2_file(path, rng, truncate=None, extra=None, drop=None):
    config = '{"architecture": "voxcpm2"}'
    tokenizer = '{"model": {"type": "BPE"}}'
    long_name = "weights/feat_decoder.estimator.decoder.layers.0.self_attn.qkv_proj.weight"
    metadata = [("general.architecture", gf.STRING, "audiocpp"),
                ("audiocpp.model_spec.family", gf.STRING, "voxcpm2"),
                ("audiocpp.tensor_names", gf.ARRAY, (gf.STRING, ["unused", long_name]))]
    metadata += gf.embedded_table({"config.json": config, "tokenizer.json": tokenizer})
    if drop is not None:
        metadata = [m for m in metadata if m[0] != drop]
    q8 = q8_tensor(rng, 64, 128)
    tensors = [("weights/base_lm.norm.weight", gf.GGML_BF16, [128],
                synth.bf16_bits(rng.normal(128).astype(np.float32)).tobytes()),
               ("_audiocpp.1", gf.GGML_Q8_0, [128, 64], q8),
               ("audiovae_weights/decoder.model.0.bias", gf.GGML_F32, [16],
                rng.normal(16).astype(np.float32).tobytes())]
    if extra is not None:
        tensors.append(extra)
    gf.write(path, metadata, tensors, truncate=truncate)
    return config, tokenizer, long_name[len("weights/"):], q8


def test_voxcpm2_layout(ops, tmp_path):
    rng = synth.Rng(62, 1)
    path = tmp_path / "voxcpm2.gguf"
    config, tokenizer, qkv_name, q8 = voxcpm2_file(path, rng)
    gguf = ops.Gguf(path)
    assert gguf.embedded("config.json") == config
    assert gguf.embedded("tokenizer.json") == tokenizer
    assert gguf.embedded("other.json") is None
    model = gguf.tensors(_lib.GGUF_MODEL)
    vae = gguf.tensors(_lib.GGUF_VAE)
    assert [t["name"] for t in model] == ["base_lm.norm.weight", qkv_name]
    assert [t["name"] for t in vae] == ["decoder.model.0.bias"]
    assert model[1]["type"] == gf.GGML_Q8_0 and model[1]["shape"] == (64, 128)
    assert model[1]["bytes"].tobytes() == q8


@pytest.mark.parametrize("case", [
    "magic", "version", "truncated-header", "truncated-data", "unsupported-type",
    "q8-partial-block", "no-component", "not-voxcpm2", "abbreviation-range",
    "bad-alignment", "nested-array", "missing-file", "byte-count-wraps"])
def test_malformed_files_fail_cleanly(ops, tmp_path, case):
    rng = synth.Rng(63, 1)
    path = tmp_path / f"{case}.gguf"
    voxcpm2 = True
    if case == "magic":
        gf.write(path, [], [], magic=b"GGUG")
    elif case == "version":
        gf.write(path, [], [], version=1)
    elif case == "truncated-header":
        voxcpm2_file(path, rng, truncate=40)
    elif case == "truncated-data":
        voxcpm2_file(path, rng)
        path.write_bytes(path.read_bytes()[:-200])
    elif case == "unsupported-type":
        voxcpm2_file(path, rng, extra=("weights/q4", 2, [32, 4], b"\0" * 72))
    elif case == "q8-partial-block":
        voxcpm2_file(path, rng, extra=("weights/q8", gf.GGML_Q8_0, [48, 2], b"\0" * 102))
    elif case == "no-component":
        voxcpm2_file(path, rng, extra=("other/x", gf.GGML_F32, [4], b"\0" * 16))
    elif case == "not-voxcpm2":
        voxcpm2_file(path, rng, drop="audiocpp.model_spec.family")
    elif case == "abbreviation-range":
        voxcpm2_file(path, rng, extra=("_audiocpp.9", gf.GGML_F32, [4], b"\0" * 16))
    elif case == "bad-alignment":
        gf.write(path, [("general.alignment", gf.U32, 48)], [])
        voxcpm2 = False
    elif case == "nested-array":
        path.write_bytes(b"GGUF" + np.array([3], "<u4").tobytes() +
                         np.array([0, 1], "<u8").tobytes() +
                         np.array([1], "<u8").tobytes() + b"k" +
                         np.array([9, 9], "<u4").tobytes() + np.array([0], "<u8").tobytes())
        voxcpm2 = False
    elif case == "missing-file":
        path = tmp_path / "absent.gguf"
    elif case == "byte-count-wraps":
        # 4 x (2^60 + 1) float32 values: 4 (2^62 + 4) bytes wrap to 16, which
        # the file holds; the tensor must still be refused.
        voxcpm2_file(path, rng, extra=("weights/huge", gf.GGML_F32, [4, 2**60 + 1], b"\0" * 16))
    with pytest.raises(_lib.VxError) as info:
        ops.Gguf(path, voxcpm2=voxcpm2)
    assert info.value.status == _lib.VX_BAD_ARG
    print(case, "->", info.value)
