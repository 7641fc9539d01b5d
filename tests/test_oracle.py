"""Pins the CPU oracle (oracle/mimi_oracle.py) before it is trusted as the
GPU parity reference.

* Reference golden vectors (tests/golden/reference_golden.npz, written by
  tests/golden/make_golden.py from kadirnar/fast-mimi itself): bit-exact.
* Hugging Face transformers.MimiModel at the reference's tiny test config —
  the oracle of the reference's own tests (tests/conftest.py:31-55): bit-exact,
  offline and streaming (padding-cache encode, KV-cache decode).
* Float64 brute force / closed forms for every primitive, each written from the
  definition (loops, explicit sums), so a dropped term, wrong sign, index shift
  or transposed operand in the oracle fails one of them.
"""

from __future__ import annotations

import hashlib
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from conftest import TINY, tiny_config, torch_state
from fast_mimi_amd import synthetic
from fast_mimi_amd.config import MimiConfig
from oracle.mimi_oracle import (
    MimiOracle,
    Trace,
    causal_conv1d,
    causal_conv_transpose1d,
    conv_output_length,
    rvq_margins,
)


@pytest.fixture(scope="module")
def tiny_oracle():
    cfg = tiny_config()
    return MimiOracle(cfg, torch_state(cfg, 1234))


@pytest.fixture(scope="module")
def full_oracle():
    cfg = MimiConfig()
    return MimiOracle(cfg, torch_state(cfg, 0))


# --------------------------------------------------------------- golden pins
@pytest.mark.parametrize("nq", [1, 2, 4])
def test_tiny_batch_matches_reference(tiny_oracle, golden, nq):
    audio = torch.from_numpy(golden[f"tiny_b2_nq{nq}_audio"])
    codes, values = tiny_oracle.forward(audio, None, nq)
    assert torch.equal(codes, torch.from_numpy(golden[f"tiny_b2_nq{nq}_codes"]).long())
    assert torch.equal(values, torch.from_numpy(golden[f"tiny_b2_nq{nq}_values"]))


@pytest.mark.parametrize("length", [1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 65, 72, 200])
def test_tiny_lengths_match_reference(tiny_oracle, golden, length):
    audio = torch.linspace(-0.1, 0.1, length).view(1, 1, -1)
    codes, values = tiny_oracle.forward(audio, None, 4)
    assert torch.equal(codes, torch.from_numpy(golden[f"tiny_len{length}_codes"]).long())
    assert torch.equal(values, torch.from_numpy(golden[f"tiny_len{length}_values"]))


def test_tiny_quantizer_decode_matches_reference(tiny_oracle, golden):
    codes = torch.from_numpy(golden["tiny_qdecode_codes"]).long()
    got = tiny_oracle.quantizer_decode(codes)
    assert torch.equal(got, torch.from_numpy(golden["tiny_qdecode_values"]))


def test_full_one_second_matches_reference(full_oracle, golden):
    audio, mask = synthetic.batch(1, 24_000)
    trace = Trace()
    codes, values = full_oracle.forward(torch.from_numpy(audio), torch.from_numpy(mask), 8, trace)
    assert torch.equal(codes, torch.from_numpy(golden["full_1s_codes"]).long())
    assert torch.equal(values, torch.from_numpy(golden["full_1s_values"]))
    assert torch.equal(trace.encoder_out, torch.from_numpy(golden["full_1s_encoder_out"]))


def test_full_padded_batch_32_codebooks_matches_reference(full_oracle, golden):
    audio, mask = synthetic.batch(2, 48_000, padded_tail=1, padded_length=28_800)
    codes, values = full_oracle.forward(torch.from_numpy(audio), torch.from_numpy(mask), 32)
    assert torch.equal(codes, torch.from_numpy(golden["full_b2_codes"]).long())
    assert torch.equal(values[..., ::10], torch.from_numpy(golden["full_b2_values_dec10"]))
    digest = hashlib.sha256(values.numpy().astype(np.float32).tobytes()).hexdigest()
    assert digest == str(golden["full_b2_values_sha256"])


def test_benchmark_c1_matches_reference(full_oracle, golden):
    audio, mask, nq = synthetic.config_inputs("c1")
    codes, values = full_oracle.forward(torch.from_numpy(audio), torch.from_numpy(mask), nq)
    assert torch.equal(codes, torch.from_numpy(golden["full_c1_codes"]).long())
    digest = hashlib.sha256(values.numpy().astype(np.float32).tobytes()).hexdigest()
    assert digest == str(golden["full_c1_values_sha256"])


def _sha(values: torch.Tensor) -> str:
    return hashlib.sha256(values.numpy().astype(np.float32).tobytes()).hexdigest()


def test_benchmark_c2_matches_reference(full_oracle, golden):
    audio, mask, nq = synthetic.config_inputs("c2")
    codes, values = full_oracle.forward(torch.from_numpy(audio), torch.from_numpy(mask), nq)
    assert torch.equal(codes, torch.from_numpy(golden["full_c2_codes"]).long())
    assert torch.equal(values[..., ::10], torch.from_numpy(golden["full_c2_values_dec10"]))
    assert _sha(values) == str(golden["full_c2_values_sha256"])
    stats = golden["full_c2_values_stats"]
    assert float(values.min()) == stats[0] and float(values.max()) == stats[1]


def test_benchmark_c3_padded_batch_matches_reference(full_oracle, golden_large):
    """Batch 16, last four clips zero-padded from 6 s (one reference call)."""
    audio, mask, nq = synthetic.config_inputs("c3")
    codes, values = full_oracle.forward(torch.from_numpy(audio), torch.from_numpy(mask), nq)
    assert torch.equal(codes, torch.from_numpy(golden_large["c3_codes"]).long())
    assert [_sha(values[c]) for c in range(16)] == golden_large["c3_values_sha256"].tolist()
    for c in (0, 12, 15):
        assert torch.equal(values[c:c + 1, :, ::10], torch.from_numpy(golden_large[f"c3_clip{c}_values_dec10"]))


def test_benchmark_c4_long_clip_matches_reference(full_oracle, golden_large):
    """100 s clip: 2,500 transformer frames through the 250-frame window."""
    audio, mask, nq = synthetic.config_inputs("c4")
    codes, values = full_oracle.forward(torch.from_numpy(audio), torch.from_numpy(mask), nq)
    assert torch.equal(codes, torch.from_numpy(golden_large["c4_codes"]).long())
    assert torch.equal(values[..., ::100], torch.from_numpy(golden_large["c4_values_dec100"]))
    assert _sha(values) == str(golden_large["c4_values_sha256"])


@pytest.mark.parametrize("clip", [0, 63])
def test_benchmark_c5_32_codebooks_matches_reference(full_oracle, golden_large, clip):
    audio, mask, nq = synthetic.config_inputs("c5")
    a, m = torch.from_numpy(audio[clip:clip + 1]), torch.from_numpy(mask[clip:clip + 1])
    codes, values = full_oracle.forward(a, m, nq)
    assert codes.shape == (1, 32, 125)
    assert torch.equal(codes, torch.from_numpy(golden_large[f"c5_clip{clip}_codes"]).long())
    assert _sha(values) == str(golden_large[f"c5_clip{clip}_values_sha256"])


def test_encoded_length_closed_form(full_oracle, golden):
    assert full_oracle.encoded_length(golden["encoded_length_in"]) == golden["encoded_length_out"].tolist()
    # Reference tests/test_config.py:45-48.
    assert full_oracle.encoded_length([1, 1919, 1920, 1921, 24000, 48001]) == [1, 1, 1, 2, 13, 26]


# ------------------------------------------------ Hugging Face oracle pin
def test_tiny_matches_transformers_mimi(tiny_oracle):
    """The reference's own test oracle: transformers.MimiModel with identical
    weights (tests/conftest.py:31-55, test_parity.py:12-53)."""
    transformers = pytest.importorskip("transformers")
    cfg = tiny_config()
    hf_cfg = transformers.MimiConfig(**cfg.to_dict())
    hf_cfg._attn_implementation = "sdpa"
    hf = transformers.MimiModel(hf_cfg).eval()
    state = torch_state(cfg, 1234)
    hf.load_state_dict(state, strict=True)
    g = torch.Generator().manual_seed(7)
    audio = torch.randn((2, 1, 65), generator=g) * 0.05
    with torch.inference_mode():
        ref = hf(audio)
    codes, values = tiny_oracle.forward(audio, None, 4)
    assert torch.equal(codes, ref.audio_codes)
    assert torch.equal(values, ref.audio_values)
    for length in (1, 9, 33, 72):
        a = torch.linspace(-0.1, 0.1, length).view(1, 1, -1)
        with torch.inference_mode():
            ref = hf(a)
        codes, values = tiny_oracle.forward(a, None, 4)
        assert torch.equal(codes, ref.audio_codes)
        assert torch.equal(values, ref.audio_values)


def _hf_model(cfg, seed):
    transformers = pytest.importorskip("transformers")
    hf_cfg = transformers.MimiConfig(**cfg.to_dict())
    hf_cfg._attn_implementation = "sdpa"
    hf = transformers.MimiModel(hf_cfg).eval()
    hf.load_state_dict(torch_state(cfg, seed), strict=True)
    return hf


@pytest.mark.parametrize("batch,samples,chunk", [(1, 40, 8), (2, 96, 16), (1, 200, 24), (1, 72, 12)])
def test_streaming_encode_matches_transformers_mimi(tiny_oracle, batch, samples, chunk):
    """Chunked encode with padding + KV caches (the reference's
    test_parity.py:56-80 scenario), bit-exact codes and cache lengths."""
    hf = _hf_model(tiny_config(), 1234)
    g = torch.Generator().manual_seed(samples)
    audio = torch.randn(batch, 1, samples, generator=g) * 0.05
    state = tiny_oracle.new_stream()
    kv = pc = None
    for piece in audio.split(chunk, dim=-1):
        codes = tiny_oracle.encode_stream(piece, 4, state)
        with torch.inference_mode():
            ref = hf.encode(piece, encoder_past_key_values=kv, padding_cache=pc, use_streaming=True)
        kv, pc = ref.encoder_past_key_values, ref.padding_cache
        assert torch.equal(codes, ref.audio_codes)
        assert state.encoder_kv.length == kv.get_seq_length()


def test_cached_decode_matches_transformers_mimi(tiny_oracle):
    """Frame-by-frame decode through the decoder KV cache, past the window
    (the reference's test_parity.py:83-110 scenario)."""
    from transformers import DynamicCache

    hf = _hf_model(tiny_config(), 1234)
    g = torch.Generator().manual_seed(99)
    kv, hc = tiny_oracle.new_kv(), DynamicCache(config=hf.config)
    for _ in range(12):
        codes = torch.randint(0, tiny_oracle.config.codebook_size, (1, 4, 1), generator=g)
        audio = tiny_oracle.decode_cached(codes, kv)
        with torch.inference_mode():
            ref = hf.decode(codes, decoder_past_key_values=hc)
        assert torch.equal(audio, ref.audio_values)
        assert kv.length == hc.get_seq_length()
        assert all(k is None or k.shape[-2] <= tiny_oracle.config.sliding_window - 1 for k in kv.keys)


def test_full_config_streaming_matches_transformers_mimi(full_oracle):
    """Full architecture: 0.4 s in 80 ms frames (1920 samples) through the streaming encoder."""
    hf = _hf_model(MimiConfig(), 0)
    audio, _ = synthetic.batch(1, 9600, base_seed=3)
    a = torch.from_numpy(audio)
    state = full_oracle.new_stream()
    kv = pc = None
    for piece in a.split(1920, dim=-1):
        codes = full_oracle.encode_stream(piece, 8, state)
        with torch.inference_mode():
            ref = hf.encode(piece, num_quantizers=8, encoder_past_key_values=kv, padding_cache=pc,
                            use_streaming=True)
        kv, pc = ref.encoder_past_key_values, ref.padding_cache
        assert torch.equal(codes, ref.audio_codes)


# -------------------------------------------------- float64 brute force
def brute_causal_conv(x, w, b, stride, pad_mode="constant"):
    """Definition: output t reads input positions t*s - (k - s) + j, j < k,
    zero (or edge) outside [0, L); ceil(L / s) outputs."""
    B, C, L = x.shape
    co, ci, k = w.shape
    T = -(-L // stride)
    y = torch.zeros(B, co, T, dtype=torch.float64)
    for t in range(T):
        for j in range(k):
            pos = t * stride - (k - stride) + j
            if pad_mode == "replicate":
                pos = min(max(pos, 0), L - 1)
            elif pos < 0 or pos >= L:
                continue
            y[:, :, t] += torch.einsum("bc,oc->bo", x[:, :, pos], w[:, :, j])
    if b is not None:
        y += b[None, :, None]
    return y


@pytest.mark.parametrize("L,k,s", [(1, 7, 1), (9, 4, 2), (10, 4, 2), (23, 8, 4), (5, 10, 5), (31, 3, 1)])
def test_conv_padding_and_stride_alignment(L, k, s):
    g = torch.Generator().manual_seed(L * k)
    x = torch.randn(2, 3, L, generator=g, dtype=torch.float64)
    w = torch.randn(4, 3, k, generator=g, dtype=torch.float64)
    b = torch.randn(4, generator=g, dtype=torch.float64)
    torch.testing.assert_close(causal_conv1d(x, w, b, s), brute_causal_conv(x, w, b, s), rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(causal_conv1d(x, w, None, s, pad_mode="replicate"),
                               brute_causal_conv(x, w, None, s, "replicate"), rtol=1e-12, atol=1e-12)
    assert conv_output_length(L, k, s) == -(-L // s)


@pytest.mark.parametrize("L,s,groups", [(1, 2, 1), (7, 4, 1), (5, 8, 1), (6, 2, 3)])
def test_conv_transpose_trim(L, s, groups):
    """out[q*s + r] = sum_j x[q - j] w[r + j*s] over q - j >= 0; L*s outputs."""
    g = torch.Generator().manual_seed(L + s)
    cin, cout = 3 * groups, 2 * groups
    x = torch.randn(1, cin, L, generator=g, dtype=torch.float64)
    w = torch.randn(cin, cout // groups, 2 * s, generator=g, dtype=torch.float64)
    got = causal_conv_transpose1d(x, w, None, s, groups)
    want = torch.zeros(1, cout, L * s, dtype=torch.float64)
    cpg_in, cpg_out = cin // groups, cout // groups
    for t in range(L * s):
        for tin in range(L):
            kk = t - tin * s
            if 0 <= kk < 2 * s:
                for gi in range(groups):
                    xs = x[0, gi * cpg_in:(gi + 1) * cpg_in, tin]
                    want[0, gi * cpg_out:(gi + 1) * cpg_out, t] += xs @ w[gi * cpg_in:(gi + 1) * cpg_in, :, kk]
    torch.testing.assert_close(got, want, rtol=1e-12, atol=1e-12)


def test_rope_tables_closed_form():
    cfg = MimiConfig()
    o = MimiOracle.__new__(MimiOracle)
    o.config = cfg
    cos, sin = o.rope_tables(1, 300)
    t = torch.arange(300, dtype=torch.float64)[:, None]
    inv = 1.0 / (cfg.rope_theta ** (torch.arange(0, 64, 2, dtype=torch.float64) / 64))
    ang = torch.cat([t * inv, t * inv], -1)
    torch.testing.assert_close(cos[0].double(), torch.cos(ang), rtol=0, atol=2e-4)
    torch.testing.assert_close(sin[0].double(), torch.sin(ang), rtol=0, atol=2e-4)
    # The float32 tables equal the runtime's (same formula, same CPU ops).
    from fast_mimi_amd.runtime import rope_tables
    rc, rs = rope_tables(cfg, 300)
    assert torch.equal(rc, cos[0]) and torch.equal(rs, sin[0])


def test_window_attention_brute_force():
    """One layer's attention through the oracle's SDPA path equals an explicit
    loop: RoPE (x*cos + rotate_half(x)*sin), scores over keys (q-W, q], softmax."""
    torch.manual_seed(0)
    cfg = MimiConfig(hidden_size=16, num_attention_heads=2, num_key_value_heads=2, head_dim=8,
                     sliding_window=5, num_hidden_layers=1)
    o = MimiOracle.__new__(MimiOracle)
    o.config = cfg
    T = 12
    q, k, v = (torch.randn(1, 2, T, 8, dtype=torch.float64) for _ in range(3))
    cos, sin = o.rope_tables(1, T)
    cos, sin = cos.double().unsqueeze(1), sin.double().unsqueeze(1)
    qr = q * cos + MimiOracle._rotate_half(q) * sin
    kr = k * cos + MimiOracle._rotate_half(k) * sin
    mask = o.attention_mask(1, T)
    got = F.scaled_dot_product_attention(qr, kr, v, attn_mask=mask, scale=1 / math.sqrt(8))
    want = torch.zeros_like(got)
    for h in range(2):
        for i in range(T):
            half = 4
            def rope(x, t):
                out = torch.empty(8, dtype=torch.float64)
                for d in range(8):
                    rot = -x[d + half] if d < half else x[d - half]
                    out[d] = x[d] * cos[0, 0, t, d] + rot * sin[0, 0, t, d]
                return out
            qi = rope(q[0, h, i], i)
            keys = [j for j in range(T) if i - 5 < j <= i]
            s = torch.stack([qi @ rope(k[0, h, j], j) / math.sqrt(8) for j in keys])
            p = torch.exp(s - s.max())
            p = p / p.sum()
            want[0, h, i] = sum(p[n] * v[0, h, j] for n, j in enumerate(keys))
    torch.testing.assert_close(got, want, rtol=1e-10, atol=1e-12)


def test_layer_norm_gelu_elu_definitions():
    x = torch.linspace(-4, 4, 101, dtype=torch.float64).view(1, 101)
    w = torch.linspace(0.5, 1.5, 101, dtype=torch.float64)
    b = torch.linspace(-1, 1, 101, dtype=torch.float64)
    mu = x.mean()
    var = ((x - mu) ** 2).mean()
    torch.testing.assert_close(F.layer_norm(x, (101,), w, b, 1e-5), (x - mu) / torch.sqrt(var + 1e-5) * w + b)
    erf = torch.tensor([math.erf(float(t) / math.sqrt(2)) for t in x[0]], dtype=torch.float64)
    torch.testing.assert_close(F.gelu(x)[0], 0.5 * x[0] * (1 + erf))
    torch.testing.assert_close(F.elu(x)[0], torch.where(x[0] > 0, x[0], torch.expm1(x[0])))


def test_cdist_mm_form_and_lowest_index_argmin():
    """nearest() = argmin over Euclidean distance, lowest index on ties."""
    g = torch.Generator().manual_seed(3)
    e = torch.randn(64, 16, generator=g)
    e[40] = e[7]  # duplicate entry: exact tie
    x = torch.cat([e[7:8] + 1e-3 * torch.randn(1, 16, generator=g), torch.randn(20, 16, generator=g)])
    got = MimiOracle.nearest(x, e)
    d = ((x.double()[:, None, :] - e.double()[None]) ** 2).sum(-1)
    want = d.argmin(-1)
    assert torch.equal(got, want)
    assert int(got[0]) == 7


def test_rvq_decode_order_is_zero_plus_left_to_right(tiny_oracle):
    codes = torch.tensor([[[1, 2], [3, 0], [2, 2], [0, 1]]])
    prefix = "quantizer.acoustic_residual_vector_quantizer"
    want = torch.zeros(())
    for j in range(3):
        want = want + tiny_oracle.embed(f"{prefix}.layers.{j}.codebook")[codes[0, j + 1]].T[None]
    proj = tiny_oracle.state[f"{prefix}.output_proj.weight"]
    want = F.conv1d(want, proj)
    sem_prefix = "quantizer.semantic_residual_vector_quantizer"
    sem = F.conv1d(torch.zeros(()) + tiny_oracle.embed(f"{sem_prefix}.layers.0.codebook")[codes[0, 0]].T[None],
                   tiny_oracle.state[f"{sem_prefix}.output_proj.weight"])
    assert torch.equal(tiny_oracle.quantizer_decode(codes), sem + want)


def test_mask_only_crops_decoded_audio(tiny_oracle):
    """Encode ignores the padding mask (model.py:3123-3134); decode crops to it."""
    audio = torch.linspace(-0.1, 0.1, 40).view(1, 1, -1)
    mask = torch.ones_like(audio, dtype=torch.bool)
    mask[..., 30:] = False
    c1, v1 = tiny_oracle.forward(audio, mask, 4)
    c2, v2 = tiny_oracle.forward(audio, None, 4)
    assert torch.equal(c1, c2) and torch.equal(v1, v2)
    short = torch.ones(1, 1, 33, dtype=torch.bool)
    assert tiny_oracle.decode(c1, short).shape[-1] == 33


def test_margins_diagnostic_runs(full_oracle):
    audio, _ = synthetic.batch(1, 24_000)
    trace = Trace()
    full_oracle.forward(torch.from_numpy(audio), None, 8, trace)
    margins = rvq_margins(full_oracle, trace)
    assert len(margins) == 8
    assert all(float(gap.min()) >= 0 for _, _, gap in margins)
