"""A Q8_0 matrix of a VoxCPM2 GGUF (the audio.cpp layout) into Q8_0 panels
on the GPU: the panels equal vx_q8_pack of the same blocks byte for byte,
and a product on them matches the oracle (error <= 1e-5 of sum |x w|),
as the reference's Uploader feeds kQ8Tiles (weights.cpp:160-186)."""
import numpy as np
import pytest
import torch

import gguf_file as gf
from voxcpm_amd import _lib, synth
from test_products_gpu import LIMIT, reference_activations, to_device

pytestmark = pytest.mark.gpu


def test_gguf_q8_upload_matches_pack_and_oracle(vx, oracle, cuda, stream, tmp_path):
    rng = synth.Rng(71, 1)
    out, inner = 2560, 1024  # the local stacks' qkv (gemm_bench.cpp:37)
    blocks = np.ascontiguousarray(synth.q8_blocks(rng, out, inner))
    metadata = [("general.architecture", gf.STRING, "audiocpp"),
                ("audiocpp.model_spec.family", gf.STRING, "voxcpm2"),
                ("audiocpp.tensor_names", gf.ARRAY, (gf.STRING, ["weights/qkv"]))]
    metadata += gf.embedded_table({"config.json": "{}", "tokenizer.json": "{}"})
    path = tmp_path / "q8.gguf"
    gf.write(path, metadata, [("_audiocpp.0", gf.GGML_Q8_0, [inner, out], blocks.tobytes())])
    gguf = vx.Gguf(path)
    packed = gguf.upload_q8("qkv", _lib.GGUF_MODEL, cuda, stream)
    expected = vx.q8_pack(torch.from_numpy(blocks).to(cuda), out, inner)
    torch.cuda.synchronize()
    assert torch.equal(packed, expected)
    for rows in (1, 22):
        x = reference_activations(rng, rows, inner)
        y = vx.q8_linear(to_device(x, cuda), packed, out)
        torch.cuda.synchronize()
        error = oracle.q8_check(y.cpu().numpy(), x, blocks.reshape(out, inner // 32, 34))
        assert error <= LIMIT, f"rows {rows}: {error:.3e}"
    with pytest.raises(_lib.VxError):  # a name the file does not hold
        gguf.upload_q8("absent", _lib.GGUF_MODEL, cuda, stream)
