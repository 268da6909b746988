"""The released-model shapes this repository tests and benchmarks
(voxcpm_amd.synth's VOXCPM2_* constants) against the released config.json,
kept as data in tests/golden/voxcpm2_config.json (written from the
reference's tests/config_samples.hpp by tests/golden/make_config_fixture.py).

Each stack's shape follows the reference's derivation (config.cpp:143-200):
the base LM from lm_config; the residual LM is the base LM with
residual_lm_num_layers layers and no rotary embedding when
residual_lm_no_rope; the local encoder and the DiT copy the base LM and
override hidden size, FFN size, heads, layers and kv_channels from their
own sections (so they keep lm_config's key/value heads and epsilon). The
rotary scale is sqrt(1 + ln(max / original) / ln(original))
(config.cpp:252-257)."""
import json
import math
import pathlib

from voxcpm_amd import synth

FIXTURE = json.loads((pathlib.Path(__file__).parent / "golden" /
                      "voxcpm2_config.json").read_text())


def derived(section: dict) -> dict:
    lm = FIXTURE["lm_config"]
    return {"hidden": section["hidden_dim"], "ffn": section["ffn_dim"],
            "heads": section["num_heads"], "layers": section["num_layers"],
            "head_dim": section["kv_channels"], "kv_heads": lm["num_key_value_heads"],
            "eps": lm["rms_norm_eps"]}


def shape_of(config) -> dict:
    return {"hidden": config.hidden, "ffn": config.ffn, "heads": config.heads,
            "layers": config.layers, "head_dim": config.head_dim,
            "kv_heads": config.kv_heads, "eps": config.eps}


def test_rope_factors_are_the_released_short_factors():
    short = FIXTURE["rope_scaling"]["short_factor"]
    assert len(synth.VOXCPM2_SHORT_FACTORS) == len(short) == 64
    assert list(synth.VOXCPM2_SHORT_FACTORS) == short  # bit for bit as float64


def test_rope_scaling_is_one():
    maximum = FIXTURE["max_position_embeddings"]
    original = FIXTURE["rope_scaling"]["original_max_position_embeddings"]
    scale = math.sqrt(1.0 + math.log(maximum / original) / math.log(original))
    for config in (synth.VOXCPM2_DIT, synth.VOXCPM2_BASE_LM, synth.VOXCPM2_ENCODER):
        assert config.rope_scaling == scale == 1.0
        assert config.rope_theta == FIXTURE["lm_config"]["rope_theta"]


def test_dit_shape():
    dit = synth.VOXCPM2_DIT
    assert shape_of(dit) == derived(FIXTURE["dit_config"])
    assert dit.patch == FIXTURE["patch_size"] and dit.feat == FIXTURE["feat_dim"]
    assert dit.rope_factors == synth.VOXCPM2_SHORT_FACTORS
    assert dit.cfg == FIXTURE["inference_cfg_rate"]


def test_lm_and_encoder_shapes():
    lm = FIXTURE["lm_config"]
    base = synth.VOXCPM2_BASE_LM
    assert shape_of(base) == {"hidden": lm["hidden_size"], "ffn": lm["intermediate_size"],
                              "heads": lm["num_attention_heads"],
                              "layers": lm["num_hidden_layers"], "head_dim": lm["kv_channels"],
                              "kv_heads": lm["num_key_value_heads"], "eps": lm["rms_norm_eps"]}
    assert base.rope and base.rope_factors == synth.VOXCPM2_SHORT_FACTORS
    residual = synth.VOXCPM2_RESIDUAL_LM
    assert residual.layers == FIXTURE["residual_lm_num_layers"]
    assert residual.rope == (not FIXTURE["residual_lm_no_rope"])
    assert {**shape_of(residual), "layers": base.layers} == shape_of(base)
    assert shape_of(synth.VOXCPM2_ENCODER) == derived(FIXTURE["encoder_config"])


def test_vae_shape():
    vae = FIXTURE["audio_vae_config"]
    config = synth.VOXCPM2_VAE
    assert config.latent == vae["latent_dim"]
    assert config.decoder_dim == vae["decoder_dim"]
    assert tuple(config.rates) == tuple(vae["decoder_rates"])
    # One latent frame decodes to the product of the rates in samples at
    # the output rate: 1920 samples at 48 kHz, 25 frames a second.
    assert config.hop == math.prod(vae["decoder_rates"]) == 1920
    assert vae["out_sample_rate"] / config.hop == 25.0
