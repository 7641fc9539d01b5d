from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest
import torch

REPO = Path(__file__).resolve().parents[1]
sys.path.insert(0, str(REPO / "fast-mimi_amd"))
sys.path.insert(0, str(REPO))

from fast_mimi_amd.config import MimiConfig  # noqa: E402
from fast_mimi_amd.weights import seeded_state_dict  # noqa: E402

GOLDEN = REPO / "tests" / "golden"

# The reference's own test configuration (tests/conftest.py:8-28 of fast-mimi).
TINY = dict(sampling_rate=64, hidden_size=16, num_filters=2, upsampling_ratios=(2, 2),
            codebook_size=16, codebook_dim=8, num_quantizers=4,
            vector_quantization_hidden_dimension=8, num_semantic_quantizers=1,
            upsample_groups=16, num_hidden_layers=2, intermediate_size=32,
            num_attention_heads=2, num_key_value_heads=2, head_dim=8,
            max_position_embeddings=128, sliding_window=8, frame_rate_override=8)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X) and the built HIP library")


def tiny_config() -> MimiConfig:
    return MimiConfig(**TINY)


def torch_state(config: MimiConfig, seed: int) -> dict[str, torch.Tensor]:
    return {k: torch.from_numpy(v) for k, v in seeded_state_dict(config, seed).items()}


@pytest.fixture(scope="session")
def golden():
    return np.load(GOLDEN / "reference_golden.npz")


@pytest.fixture(scope="session")
def golden_large():
    """Reference outputs of the larger benchmark configurations (C3, C4, C5 clips)
    and of ``get_audio_codes_mask``."""
    return np.load(GOLDEN / "reference_golden_large.npz")


def gpu_available() -> bool:
    return torch.cuda.is_available()
