"""AudioVAE V2's streaming decoder (vx_vae) on the GPU against the CPU
oracle's whole-sequence decode (vae.cpp:415-481; the reference's
vae_test compares streamed and at-once decoding, vae_test.cpp:114-138):
chunks of latents decoded in turn equal the whole sequence decoded at
once; a reset starts a new stream; graph replays with the same buffers
match. Tolerance: float32 products in another summation order through
the decoder's 25 layers and Snake on the hardware sine, max |gpu -
oracle| <= 2e-3 on samples in [-1, 1] (measured 5.1e-6 small, 7.7e-4 at
the VoxCPM2 shape)."""
import numpy as np
import pytest
import torch

from voxcpm_amd import _lib, synth

pytestmark = pytest.mark.gpu

BOUND = 2e-3

# "small" and "odd" take channel counts that are not multiples of 16 (8;
# 24 and 12): their products go to the LDS-tiled float32 kernel
# (F32TileKernel), whose epilogue makes the next inputs (unit windows, a
# block's input, the output window) as the 16-column kernel's does. Units
# of at most 256 channels (and the latents' input convolutions) make their
# depthwise convolution in the pointwise product's operand loads; chunks
# of 1, 5 and 2 frames at the VoxCPM2 shape take one- and two-tile row
# blocks and latents' histories that mix the previous chunk's rows with
# this chunk's (fewer than 6 frames).
# "split": a transposed convolution of k = 2080 over 1560 columns at a
# few rows splits k over 32 x 32 tiles (the last column tile partial) and a
# second launch adds the splits; its 520-channel units take depthwise
# launches and the LDS-tiled kernel (520 is not a multiple of 16).
CONFIGS = {
    "small": synth.VaeConfig(latent=16, decoder_dim=64, rates=(3, 2, 2)),
    "odd": synth.VaeConfig(latent=16, decoder_dim=48, rates=(2, 2)),
    "split": synth.VaeConfig(latent=16, decoder_dim=1040, rates=(3,)),
    "voxcpm2": synth.VOXCPM2_VAE,
}


@pytest.mark.parametrize("name,chunks", [("small", (4, 4, 1)), ("small", (9,)),
                                         ("odd", (3, 2, 5)), ("split", (4, 3, 1)),
                                         ("voxcpm2", (4, 4)), ("voxcpm2", (1, 5, 2))])
def test_vae_streaming_decode_against_oracle(vx, oracle, cuda, stream, name, chunks):
    config = CONFIGS[name]
    weights = synth.vae_weights(config, 91)
    frames = sum(chunks)
    rng = synth.Rng(92, frames)
    latents = rng.normal(frames * config.latent).astype(np.float32).reshape(frames, config.latent)
    ref = oracle.OracleVae(weights).decode(latents)
    vae = vx.Vae(weights)
    assert vae.hop == config.hop
    device_latents = torch.from_numpy(latents).to(cuda)
    for attempt in range(2):  # the second stream after a reset
        pieces, at = [], 0
        for n in chunks:
            pieces.append(vae.decode(device_latents[at:at + n]).cpu().numpy())
            at += n
        got = np.concatenate(pieces)
        error = float(np.max(np.abs(got - ref)))
        print(f"{name} {chunks} stream {attempt}: max |d| {error:.2e}, "
              f"signal std {np.std(ref):.3f}", flush=True)
        assert error <= BOUND
        vae.reset()


def test_vae_graph_replays(vx, oracle, cuda, stream):
    """One chunk buffer decoded again and again (the patch loop): the first
    call runs eagerly, later ones replay one graph; every chunk matches the
    oracle's decode of the whole sequence so far."""
    config = CONFIGS["small"]
    weights = synth.vae_weights(config, 93)
    rng = synth.Rng(94, 1)
    latents = rng.normal(5 * 4 * config.latent).astype(np.float32).reshape(20, config.latent)
    ref = oracle.OracleVae(weights).decode(latents)
    vae = vx.Vae(weights)
    chunk = torch.empty((4, config.latent), dtype=torch.float32, device=cuda)
    samples = torch.empty(4 * config.hop, dtype=torch.float32, device=cuda)
    for i in range(5):
        chunk.copy_(torch.from_numpy(latents[4 * i:4 * i + 4]))
        vae.decode(chunk, samples)
        got = samples.cpu().numpy()
        want = ref[4 * i * config.hop:4 * (i + 1) * config.hop]
        assert float(np.max(np.abs(got - want))) <= BOUND, i


def test_vae_chunk_limit(vx, cuda):
    """A chunk of more frames than vx_vae_max_frames is refused before any
    launch (a product's 32-row blocks are grid rows, at most 65535)."""
    config = CONFIGS["small"]
    vae = vx.Vae(synth.vae_weights(config, 95))
    assert vae.max_frames == 65535 * 32 // config.hop
    latents = torch.zeros((vae.max_frames + 1, config.latent), dtype=torch.float32, device=cuda)
    with pytest.raises(_lib.VxError) as info:
        vae.decode(latents)
    assert info.value.status == _lib.VX_BAD_ARG


def test_vae_longest_chunk(vx, cuda):
    """A chunk of vx_vae_max_frames frames at the VoxCPM2 shape (1092: its
    32-row blocks fill the grid's 65535 rows at the output rate) decodes,
    and equals the same latents decoded in chunks of 16 frames (vae.cpp
    streams chunk by chunk; the two take different tilings, so the bound is
    the oracle tolerance)."""
    config = CONFIGS["voxcpm2"]
    weights = synth.vae_weights(config, 97)
    whole = vx.Vae(weights)
    frames = whole.max_frames
    assert frames == 65535 * 32 // config.hop
    rng = synth.Rng(98, frames)
    latents = torch.from_numpy(
        rng.normal(frames * config.latent).astype(np.float32).reshape(frames, config.latent)
    ).to(cuda)
    print(f"longest chunk: {frames} frames", flush=True)
    at_once = whole.decode(latents).cpu().numpy()
    chunked = vx.Vae(weights)
    pieces = [chunked.decode(latents[at:at + 16]).cpu().numpy() for at in range(0, frames, 16)]
    error = float(np.max(np.abs(at_once - np.concatenate(pieces))))
    print(f"longest chunk against 16-frame chunks: max |d| {error:.2e}", flush=True)
    assert np.all(np.isfinite(at_once))
    assert error <= BOUND


def test_vae_decode_argument_checks(vx, cuda):
    """The C ABI takes bare pointers: Vae.decode refuses tensors whose bytes
    are not float32 [frames][latent] rows (bf16, strided, wrong width) and
    sample buffers too small for the chunk, before any launch."""
    config = CONFIGS["small"]
    vae = vx.Vae(synth.vae_weights(config, 96))
    good = torch.zeros((4, config.latent), dtype=torch.float32, device=cuda)
    bad = [good.to(torch.bfloat16),
           torch.zeros((config.latent, 8), dtype=torch.float32, device=cuda).t()[:4],
           torch.zeros((4, config.latent + 1), dtype=torch.float32, device=cuda),
           good.reshape(-1)]
    for latents in bad:
        with pytest.raises(ValueError):
            vae.decode(latents)
    with pytest.raises(ValueError):
        vae.decode(good, torch.empty(4 * config.hop - 1, dtype=torch.float32, device=cuda))
    vae.decode(good, torch.empty(4 * config.hop, dtype=torch.float32, device=cuda))
    torch.cuda.synchronize()
