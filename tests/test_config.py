"""Configuration, checkpoint layout and seeded-initialisation tests
(mirroring kadirnar/fast-mimi tests/test_config.py)."""

from __future__ import annotations

import ast
import json
from pathlib import Path

import numpy as np
import pytest
import torch

import fast_mimi_amd
from conftest import GOLDEN, TINY
from fast_mimi_amd import (
    KYUTAI_MIMI_MODEL_ID,
    KYUTAI_MIMI_PARAMETER_COUNT,
    KYUTAI_MIMI_PARAMETER_FINGERPRINT,
    KYUTAI_MIMI_REVISION,
    KYUTAI_MIMI_WEIGHTS_SHA256,
    MimiConfig,
    MimiModel,
)
from fast_mimi_amd.weights import parameter_count, seeded_state_dict, state_dict_spec


def test_published_defaults() -> None:
    config = MimiConfig()
    assert KYUTAI_MIMI_MODEL_ID == "kyutai/mimi"
    assert KYUTAI_MIMI_REVISION == "89091b3e466eb6a9d11e537bf26b144f194978f7"
    assert KYUTAI_MIMI_PARAMETER_COUNT == 79_308_609
    assert len(KYUTAI_MIMI_PARAMETER_FINGERPRINT) == 64
    assert len(KYUTAI_MIMI_WEIGHTS_SHA256) == 64
    assert config.sampling_rate == 24_000
    assert config.frame_rate == 12.5
    assert config.encodec_frame_rate == 25
    assert config.frame_size == 1_920
    assert config.num_codebooks == 32
    assert config.codebook_size == 2_048


def test_json_round_trip_maps_frame_rate(tmp_path) -> None:
    config = MimiConfig()
    path = config.save_pretrained(tmp_path)
    loaded = MimiConfig.from_json_file(path)
    assert loaded == config
    assert json.loads(path.read_text())["frame_rate"] == 12.5


def test_encoded_lengths_match_frame_boundaries() -> None:
    model = MimiModel(MimiConfig())
    lengths = torch.tensor([1, 1_919, 1_920, 1_921, 24_000, 48_001])
    assert model.get_encoded_length(lengths).tolist() == [1, 1, 1, 2, 13, 26]


def test_audio_codes_mask() -> None:
    model = MimiModel(MimiConfig())
    mask = torch.zeros(2, 48_000, dtype=torch.bool)
    mask[0, :] = True
    mask[1, :24_000] = True
    codes_mask = model.get_audio_codes_mask(mask)
    assert codes_mask.shape == (2, 25)
    assert codes_mask[0].all() and codes_mask[1].sum() == 13
    assert torch.equal(model.get_audio_codes_mask(mask, "left"), codes_mask.flip(-1))


def test_invalid_quantizer_split_is_rejected() -> None:
    with pytest.raises(ValueError, match="num_semantic_quantizers"):
        MimiConfig(num_quantizers=1, num_semantic_quantizers=1)


def test_declared_checkpoint_revision_is_locked() -> None:
    with pytest.raises(ValueError, match="revision changed"):
        MimiModel.from_pretrained(KYUTAI_MIMI_MODEL_ID, revision="main", local_files_only=True)


def test_runtime_has_no_transformers_import() -> None:
    package = Path(fast_mimi_amd.__file__).parent
    for source_path in package.glob("*.py"):
        tree = ast.parse(source_path.read_text(), filename=str(source_path))
        names = [n.module for n in ast.walk(tree) if isinstance(n, ast.ImportFrom) and n.module]
        names += [a.name for n in ast.walk(tree) if isinstance(n, ast.Import) for a in n.names]
        assert all(not name.startswith("transformers") for name in names), source_path
        assert all(not name.startswith("oracle") for name in names), source_path


def test_state_layout_matches_reference() -> None:
    """Names, order and shapes equal the reference's state_dict (fixture)."""
    layout = json.loads((GOLDEN / "reference_state_layout.json").read_text())
    spec = state_dict_spec(MimiConfig())
    assert [s.name for s in spec] == [name for name, _ in layout]
    assert [list(s.shape) for s in spec] == [shape for _, shape in layout]
    assert parameter_count(MimiConfig()) == KYUTAI_MIMI_PARAMETER_COUNT


def test_seeded_weights_are_deterministic_and_follow_the_init_scheme() -> None:
    cfg = MimiConfig(**TINY)
    a, b = seeded_state_dict(cfg, 3), seeded_state_dict(cfg, 3)
    assert all(np.array_equal(a[k], b[k]) for k in a)
    c = seeded_state_dict(cfg, 4)
    assert not np.array_equal(a["encoder.layers.0.conv.weight"], c["encoder.layers.0.conv.weight"])
    full = seeded_state_dict(MimiConfig(), 0)
    w = full["encoder.layers.3.conv.weight"]  # Kaiming normal, fan_in = 64 * 8
    assert abs(w.std() - (2.0 / (64 * 8)) ** 0.5) < 0.01 * (2.0 / 512) ** 0.5 * 10
    e = full["quantizer.acoustic_residual_vector_quantizer.layers.3.codebook.embed_sum"]
    assert abs(e.std() - 1 / 16) < 1e-3
    assert (full["decoder_transformer.layers.2.mlp_layer_scale.scale"] == 0.01).all()
    assert (full["encoder_transformer.layers.0.input_layernorm.weight"] == 1).all()


def test_save_and_load_round_trip(tmp_path) -> None:
    cfg = MimiConfig(**TINY)
    model = MimiModel(cfg, seed=5)
    model.save_pretrained(tmp_path)
    loaded = MimiModel.from_pretrained(tmp_path)
    assert loaded.config == cfg
    sa, sb = model.state_dict(), loaded.state_dict()
    assert list(sa) == list(sb) and all(torch.equal(sa[k], sb[k]) for k in sa)


def test_strict_load_rejects_missing_and_mismatched() -> None:
    model = MimiModel(MimiConfig(**TINY))
    state = model.state_dict()
    broken = dict(state)
    broken.pop("encoder.layers.0.conv.weight")
    with pytest.raises(RuntimeError, match="missing"):
        model.load_state_dict(broken)
    bad = dict(state)
    bad["encoder.layers.0.conv.bias"] = torch.zeros(3)
    with pytest.raises(RuntimeError, match="size mismatch"):
        model.load_state_dict(bad)
