"""MimiModel surface on the CPU: validation errors, output containers and the
no-fallback rule (the model computes only on a ROCm GPU)."""

from __future__ import annotations

import pytest
import torch

from conftest import TINY
from fast_mimi_amd import MimiConfig, MimiModel, MimiOutput


def test_cpu_model_refuses_to_run_without_gpu():
    model = MimiModel(MimiConfig(**TINY))
    with pytest.raises(RuntimeError, match="ROCm GPU"):
        model(torch.zeros(1, 1, 64))


def test_validation_errors_precede_execution():
    model = MimiModel(MimiConfig(**TINY))
    with pytest.raises(ValueError, match="num_quantizers"):
        model(torch.zeros(1, 1, 64), num_quantizers=5)
    with pytest.raises(ValueError, match="num_quantizers"):
        model.encode(torch.zeros(1, 1, 64), num_quantizers=0)
    with pytest.raises(ValueError, match="shape"):
        model.encode(torch.zeros(1, 64))
    with pytest.raises(ValueError, match="channels"):
        model.encode(torch.zeros(1, 3, 64))
    with pytest.raises(NotImplementedError, match="streaming"):
        model.encode(torch.zeros(1, 1, 64), use_streaming=True)
    with pytest.raises(ValueError, match="attention_backend"):
        MimiModel(MimiConfig(**TINY), attention_backend="flash")


def test_output_container_behaves_like_model_output():
    codes, audio = torch.zeros(1, 2, 3), torch.ones(1, 1, 4)
    out = MimiOutput(codes, audio)
    assert len(out) == 2 and out[0] is codes and out["audio_values"] is audio
    a, b = out
    assert a is codes and b is audio
    assert out.get("encoder_past_key_values") is None
    assert out.get("missing", 7) == 7


def test_fp32_only():
    with pytest.raises(ValueError, match="float32"):
        MimiModel(MimiConfig(**TINY)).to(dtype=torch.float16)
