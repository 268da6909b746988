"""Writes tests/golden/voxcpm2_config.json: the fields of the released
VoxCPM2 config.json that this repository's released-model shapes rest on,
read from the reference's config sample (tests/config_samples.hpp:6-220,
openbmb/VoxCPM2's config.json re-serialized as a C++ raw string).

    python tests/golden/make_config_fixture.py [reference root]

Only data is kept: the numbers, not the reference's text. The derivation of
each stack's shape from them (config.cpp:143-200) is restated in
tests/test_config_fixture.py, which compares voxcpm_amd.synth's constants
with this file.
"""
from __future__ import annotations

import json
import pathlib
import sys

HERE = pathlib.Path(__file__).resolve().parent


def extract(header: str) -> dict:
    start = header.index('R"json(') + len('R"json(')
    end = header.index(')json"', start)
    return json.loads(header[start:end])


def main() -> None:
    root = pathlib.Path(sys.argv[1] if len(sys.argv) > 1 else "/root/reference")
    config = extract((root / "tests" / "config_samples.hpp").read_text())
    lm = config["lm_config"]
    keep = {
        "source": "tests/config_samples.hpp (openbmb/VoxCPM2 config.json)",
        "lm_config": {key: lm[key] for key in (
            "hidden_size", "intermediate_size", "num_attention_heads", "num_hidden_layers",
            "num_key_value_heads", "rms_norm_eps", "rope_theta", "kv_channels")},
        "rope_scaling": {key: lm["rope_scaling"][key] for key in (
            "type", "short_factor", "long_factor", "original_max_position_embeddings")},
        "max_position_embeddings": lm["max_position_embeddings"],
        "patch_size": config["patch_size"],
        "feat_dim": config["feat_dim"],
        "residual_lm_num_layers": config["residual_lm_num_layers"],
        "residual_lm_no_rope": config["residual_lm_no_rope"],
        "encoder_config": config["encoder_config"],
        "dit_config": {key: config["dit_config"][key] for key in (
            "hidden_dim", "ffn_dim", "num_heads", "num_layers", "kv_channels")},
        "inference_cfg_rate": config["dit_config"]["cfm_config"]["inference_cfg_rate"],
        "audio_vae_config": {key: config["audio_vae_config"][key] for key in (
            "latent_dim", "decoder_dim", "decoder_rates", "out_sample_rate")},
    }
    out = HERE / "voxcpm2_config.json"
    out.write_text(json.dumps(keep, indent=1) + "\n")
    print(f"wrote {out}")


if __name__ == "__main__":
    main()
