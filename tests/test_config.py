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


@pytest.mark.parametrize("side", ["right", "left"])
@pytest.mark.parametrize("ndim", [2, 3])
def test_audio_codes_mask_matches_reference(golden_large, ndim, side) -> None:
    """2-D masks give [B, T]; 3-D [B, 1, S] masks broadcast to [B, B, T] as the
    reference's do (model.py:3040-3044); fixtures from the reference itself."""
    model = MimiModel(MimiConfig())
    mask = torch.from_numpy(golden_large["codes_mask_in_2d"])
    if ndim == 3:
        mask = mask[:, None]
    got = model.get_audio_codes_mask(mask, side)
    want = torch.from_numpy(golden_large[f"codes_mask_{ndim}d_{side}"])
    assert got.dtype == torch.bool and torch.equal(got, want)


def _hub_cache(root: Path, repo_id: str, commit: str, config: MimiConfig, weights: bytes | None,
               model: MimiModel | None = None) -> None:
    """The huggingface_hub cache layout: refs/main -> commit, snapshots/<commit>/files."""
    repo = root / ("models--" + repo_id.replace("/", "--"))
    snap = repo / "snapshots" / commit
    snap.mkdir(parents=True)
    (repo / "refs").mkdir()
    (repo / "refs" / "main").write_text(commit)
    config.save_pretrained(snap)
    if model is not None:
        model.save_pretrained(snap)
    else:
        (snap / "model.safetensors").write_bytes(weights)


def test_hub_id_resolves_through_local_cache(tmp_path) -> None:
    """A Hub repository id loads from an existing cache with local_files_only
    (model.py:2898-2920); no network access is attempted."""
    cfg = MimiConfig(**TINY)
    model = MimiModel(cfg, seed=9)
    commit = "0123456789abcdef0123456789abcdef01234567"
    _hub_cache(tmp_path, "someone/mimi-tiny", commit, cfg, None, model)
    for rev in ("main", commit):
        loaded = MimiModel.from_pretrained("someone/mimi-tiny", revision=rev, cache_dir=tmp_path,
                                           local_files_only=True)
        assert loaded.config == cfg
        sa, sb = model.state_dict(), loaded.state_dict()
        assert all(torch.equal(sa[k], sb[k]) for k in sa)
    with pytest.raises(OSError):  # not cached, and the network may not be used
        MimiModel.from_pretrained("someone/absent", revision="main", cache_dir=tmp_path,
                                  local_files_only=True)


def test_declared_checkpoint_config_and_digest_are_locked(tmp_path) -> None:
    """kyutai/mimi keeps its identity locks through the cache: drifted declared
    config fields fail first (model.py:92-100), then a changed weights digest."""
    drifted = MimiConfig(frame_rate_override=25.0)
    _hub_cache(tmp_path / "a", KYUTAI_MIMI_MODEL_ID, KYUTAI_MIMI_REVISION, drifted, b"not the weights")
    with pytest.raises(RuntimeError, match="declared checkpoint config 'frame_rate' changed"):
        MimiModel.from_pretrained(KYUTAI_MIMI_MODEL_ID, cache_dir=tmp_path / "a", local_files_only=True)
    _hub_cache(tmp_path / "b", KYUTAI_MIMI_MODEL_ID, KYUTAI_MIMI_REVISION, MimiConfig(), b"not the weights")
    with pytest.raises(RuntimeError, match="digest changed"):
        MimiModel.from_pretrained(KYUTAI_MIMI_MODEL_ID, cache_dir=tmp_path / "b", local_files_only=True)
