"""Write reference golden vectors for the oracle tests.

Runs the reference implementation (kadirnar/fast-mimi, mounted read-only at
``/root/reference``) on the CPU, in the build container only, with this
repository's seeded weights and seeded synthetic audio, and stores its outputs
as small ``.npz`` fixtures next to this script.  Nothing at test time imports
the reference; the fixtures are data: inputs, codes, waveforms (full or
decimated plus a SHA-256 of the full float32 bytes) and the checkpoint layout.

Usage:  python tests/golden/make_golden.py [/root/reference/src] [--large-only]

``reference_golden.npz`` holds the small configurations; the larger
benchmark configurations (batch 16 with a padded tail, the 100 s clip, the
32-codebook clips) and ``get_audio_codes_mask`` outputs go to
``reference_golden_large.npz``.
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
ARGS = [a for a in sys.argv[1:] if not a.startswith("--")]
sys.path.insert(0, ARGS[0] if ARGS else "/root/reference/src")

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


def large(full) -> None:
    """Benchmark configurations C3-C5 and the frame-mask helper."""
    out: dict[str, np.ndarray] = {}
    # C3: the whole padded batch of 16 in one reference call.
    a, m, nq = synthetic.config_inputs("c3")
    codes, wave = run(full, a, m, nq)
    out["c3_codes"] = codes
    for c in (0, 12, 15):
        out[f"c3_clip{c}_values_dec10"] = wave[c:c + 1, :, ::10]
    out["c3_values_sha256"] = np.array([sha(wave[c]) for c in range(wave.shape[0])])
    # C4: one 100 s clip.
    a, m, nq = synthetic.config_inputs("c4")
    codes, wave = run(full, a, m, nq)
    out["c4_codes"], out["c4_values_dec100"] = codes, wave[..., ::100]
    out["c4_values_sha256"] = np.array(sha(wave))
    # C5 (32 codebooks): its first and last clips, each as a batch of one.
    a, m, nq = synthetic.config_inputs("c5")
    for c in (0, 63):
        codes, wave = run(full, a[c:c + 1], m[c:c + 1], nq)
        out[f"c5_clip{c}_codes"], out[f"c5_clip{c}_values_dec10"] = codes, wave[..., ::10]
        out[f"c5_clip{c}_values_sha256"] = np.array(sha(wave))
    # get_audio_codes_mask on 2-D and 3-D sample masks, both padding sides.
    lengths = [24_000, 1_921, 17, 0]
    mask2 = np.zeros((len(lengths), 24_000), dtype=bool)
    for i, n in enumerate(lengths):
        mask2[i, :n] = True
    out["codes_mask_in_2d"] = mask2
    for side in ("right", "left"):
        out[f"codes_mask_2d_{side}"] = full.get_audio_codes_mask(torch.from_numpy(mask2), side).numpy()
        out[f"codes_mask_3d_{side}"] = full.get_audio_codes_mask(
            torch.from_numpy(mask2[:, None]), side).numpy()
    np.savez_compressed(HERE / "reference_golden_large.npz", **out)
    print("wrote", len(out), "large arrays")


def main() -> None:
    torch.manual_seed(0)
    if "--large-only" in sys.argv:
        large(build({}, 0))
        return
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
    large(full)

    layout = [[k, list(v.shape)] for k, v in full.state_dict().items()]
    (HERE / "reference_state_layout.json").write_text(json.dumps(layout) + "\n")
    print("wrote", len(out), "arrays;", len(layout), "state entries")


if __name__ == "__main__":
    main()
