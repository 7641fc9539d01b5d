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


def test_kv_cache_window_and_positions():
    """MimiKVCache semantics (model.py:363-518): window - 1 frames retained,
    cumulative positions unbounded, mask sizes as _attention_mask needs them."""
    from fast_mimi_amd import MimiKVCache

    kv = MimiKVCache(2, sliding_window=4)
    assert kv.get_seq_length() == 0 and kv.get_mask_sizes(2) == (2, 0)
    for step in range(1, 6):
        k = torch.full((1, 2, 3), float(step))
        keys, values = kv.update(k, -k, 0)
        assert kv.get_seq_length(0) == 2 * step
        assert keys.shape[1] == min(2 * step - 2, 3) + 2        # stored + new frames
        assert kv.key_cache[0].shape[1] == min(2 * step, 3)      # window - 1 kept
        assert torch.equal(kv.value_cache[0], -kv.key_cache[0])
    # 10 frames seen: keys visible to 2 more queries are the last 3 stored + 2 new.
    assert kv.get_mask_sizes(2) == (5, 7)
    assert kv.get_seq_length(1) == 0 and kv.get_seq_length(9) == 0
    kv.update(torch.zeros(1, 1, 3), torch.zeros(1, 1, 3), 5)      # grows lazily
    assert len(kv.key_cache) == 6
    with pytest.raises(ValueError):
        MimiKVCache(1, sliding_window=0)
    with pytest.raises(ValueError, match="match"):
        kv.configure_sliding_window(8)
    late = MimiKVCache(1)
    late.update(torch.arange(12.0).view(1, 6, 2), torch.zeros(1, 6, 2), 0)
    late.configure_sliding_window(3)
    assert late.key_cache[0].shape[1] == 2 and late.get_seq_length() == 6
    assert torch.equal(late.key_cache[0], torch.arange(8.0, 12.0).view(1, 2, 2))


def test_padding_cache_context_rules():
    """MimiConv1dPaddingCache.update (model.py:536-620): zero or replicated
    first context; the newest `padding` rows (of context + chunk) are kept."""
    from fast_mimi_amd import MimiConv1dPaddingCache

    pc = MimiConv1dPaddingCache(3, [3, 2, 0], ["constant", "replicate", "constant"], [1, 2, 4])
    x = torch.arange(1.0, 3.0).view(1, 2, 1)                        # 2 rows < padding 3
    assert torch.equal(pc.update(x, 0), torch.zeros(1, 3, 1))
    assert torch.equal(pc.padding_cache[0].flatten(), torch.tensor([0.0, 1.0, 2.0]))
    x2 = torch.arange(3.0, 8.0).view(1, 5, 1)
    assert torch.equal(pc.update(x2, 0).flatten(), torch.tensor([0.0, 1.0, 2.0]))
    assert torch.equal(pc.padding_cache[0].flatten(), torch.tensor([5.0, 6.0, 7.0]))
    y = torch.tensor([[[4.0, 5.0], [6.0, 7.0], [8.0, 9.0]]])
    assert torch.equal(pc.update(y, 1), torch.tensor([[[4.0, 5.0], [4.0, 5.0]]]))
    assert torch.equal(pc.padding_cache[1], y[:, 1:])
    assert pc.update(torch.ones(1, 3, 4), 2).shape == (1, 0, 4)
    with pytest.raises(ValueError):
        MimiConv1dPaddingCache(2, [1], ["constant"], [1])
    with pytest.raises(NotImplementedError):
        MimiConv1dPaddingCache(1, [1], ["reflect"], [1])


def test_bf16x6_weight_plan_for_the_mimi_config():
    """Every SEANet conv but the 1-channel first conv (K = 7) and every
    transformer projection carries bf16x6 planes in the published config; the
    runtime raises if the layers it built differ from this plan."""
    from fast_mimi_amd.runtime import x6_plan

    cfg = MimiConfig()
    plan = x6_plan(cfg)
    assert [n for n, on in plan.items() if not on] == ["enc.first"]
    convs = {n for n in plan if not n.startswith(("enc.tf", "dec.tf"))}
    assert convs == {"enc.first", "enc.res64.c1", "enc.res64.c2", "enc.down4", "enc.res128.c1",
                     "enc.res128.c2", "enc.down5", "enc.res256.c1", "enc.res256.c2", "enc.down6",
                     "enc.res512.c1", "enc.res512.c2", "enc.down8", "enc.last", "down", "dec.first",
                     "dec.up8", "dec.res512.c1", "dec.res512.c2", "dec.up6", "dec.res256.c1",
                     "dec.res256.c2", "dec.up5", "dec.res128.c1", "dec.res128.c2", "dec.up4",
                     "dec.res64.c1", "dec.res64.c2", "dec.last"}
    projections = [n for n in plan if n.startswith(("enc.tf", "dec.tf"))]
    assert len(projections) == 2 * cfg.num_hidden_layers * 4
    # A reduction length that is not a multiple of 16 falls out of the plan.
    odd = x6_plan(MimiConfig(**{**TINY, "hidden_size": 24, "intermediate_size": 40}))
    assert odd["enc.tf0.fc2"] is False and odd["enc.tf0.qkv"] is False
