"""Write reference golden vectors for the oracle tests.

Runs the reference implementation (kadirnar/fast-mimi, mounted read-only at
``/root/reference``) on the CPU, in the build container only, with this
repository's seeded weights and seeded synthetic audio, and stores its outputs
as small ``.npz`` fixtures next to this script.  Nothing at test time imports
the reference; the fixtures are data: inputs, codes, waveforms (full or
decimated plus a SHA-256 of the full float32 bytes) and the checkpoint layout.

Usage:  python tests/golden/make_golden.py [/root/reference/src]
"""

from __future__ import annotations

import hashlib
import json
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REPO = HERE.parents[1]
sys.path.insert(0, str(REPO / "fast-mimi_amd"))
sys.path.insert(0, sys.argv[1] if len(sys.argv) > 1 else "/root/reference/src")

import fast_mimi as reference  # noqa: E402  (the reference package)
from fast_mimi_amd import synthetic  # noqa: E402
from fast_mimi_amd.config import MimiConfig  # noqa: E402
from fast_mimi_amd.weights import seeded_state_dict  # noqa: E402

TINY = dict(sampling_rate=64, hidden_size=16, num_filters=2, upsampling_ratios=(2, 2),
            codebook_size=16, codebook_dim=8, num_quantizers=4,
            vector_quantization_hidden_dimension=8, num_semantic_quantizers=1,
            upsample_groups=16, num_hidden_layers=2, intermediate_size=32,
            num_attention_heads=2, num_key_value_heads=2, head_dim=8,
            max_position_embeddings=128, sliding_window=8, frame_rate_override=8)


def build(config_kwargs: dict, seed: int):
    config = reference.MimiConfig(**config_kwargs)
    model = reference.MimiModel(config).eval()
    mine = seeded_state_dict(MimiConfig(**config_kwargs), seed)
    state = {k: torch.from_numpy(v) for k, v in mine.items()}
    model.load_state_dict(state, strict=True)
    return model


def run(model, audio: np.ndarray, mask: np.ndarray | None, nq: int):
    with torch.inference_mode():
        out = model(torch.from_numpy(audio),
                    None if mask is None else torch.from_numpy(mask),
                    num_quantizers=nq)
    return out.audio_codes.numpy().astype(np.int16), out.audio_values.numpy().astype(np.float32)


def sha(a: np.ndarray) -> str:
    return hashlib.sha256(np.ascontiguousarray(a, dtype=np.float32).tobytes()).hexdigest()


def main() -> None:
    torch.manual_seed(0)
    out: dict[str, np.ndarray] = {}

    # ---- tiny config (the reference's own test config) ----
    tiny = build(TINY, 1234)
    rng = np.random.Generator(np.random.PCG64(7))
    audio = (rng.standard_normal((2, 1, 65)) * 0.05).astype(np.float32)
    for nq in (1, 2, 4):
        codes, wave = run(tiny, audio, None, nq)
        out[f"tiny_b2_nq{nq}_audio"] = audio
        out[f"tiny_b2_nq{nq}_codes"] = codes
        out[f"tiny_b2_nq{nq}_values"] = wave
    for length in (1, 2, 3, 4, 5, 7, 8, 9, 15, 16, 17, 31, 32, 33, 65, 72, 200):
        a = np.linspace(-0.1, 0.1, length, dtype=np.float32).reshape(1, 1, -1)
        codes, wave = run(tiny, a, None, 4)
        out[f"tiny_len{length}_codes"] = codes
        out[f"tiny_len{length}_values"] = wave
    # Decode-only: ordered gather-sum of hand-picked codes.
    codes = torch.tensor([[[0, 1, 2], [3, 2, 1], [1, 0, 3], [2, 3, 0]]])
    with torch.inference_mode():
        out["tiny_qdecode_codes"] = codes.numpy().astype(np.int16)
        out["tiny_qdecode_values"] = tiny.quantizer.decode(codes).numpy()

    # ---- full-size config, seeded weights ----
    full = build({}, 0)
    out["encoded_length_in"] = np.array([1, 1919, 1920, 1921, 24000, 48001], dtype=np.int64)
    out["encoded_length_out"] = full.get_encoded_length(
        torch.from_numpy(out["encoded_length_in"])).numpy()

    a, m = synthetic.batch(1, 24_000)
    codes, wave = run(full, a, m, 8)
    out["full_1s_codes"], out["full_1s_values"] = codes, wave
    with torch.inference_mode():
        emb = full.encoder(torch.from_numpy(a))
        out["full_1s_encoder_out"] = emb.numpy()

    a, m = synthetic.batch(2, 48_000, padded_tail=1, padded_length=28_800)
    codes, wave = run(full, a, m, 32)
    out["full_b2_codes"], out["full_b2_values_dec10"] = codes, wave[..., ::10]
    out["full_b2_values_sha256"] = np.array(sha(wave))

    for name in ("c1", "c2"):
        a, m, nq = synthetic.config_inputs(name)
        codes, wave = run(full, a, m, nq)
        out[f"full_{name}_codes"] = codes
        out[f"full_{name}_values_dec10"] = wave[..., ::10]
        out[f"full_{name}_values_sha256"] = np.array(sha(wave))
        out[f"full_{name}_values_stats"] = np.array(
            [wave.min(), wave.max(), float(np.sqrt(np.mean(wave.astype(np.float64) ** 2)))])

    np.savez_compressed(HERE / "reference_golden.npz", **out)

    layout = [[k, list(v.shape)] for k, v in full.state_dict().items()]
    (HERE / "reference_state_layout.json").write_text(json.dumps(layout) + "\n")
    print("wrote", len(out), "arrays;", len(layout), "state entries")


if __name__ == "__main__":
    main()
