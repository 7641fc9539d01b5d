"""Mimi codec configuration (checkpoint-compatible field names).

Mirrors the public ``MimiConfig`` of kadirnar/fast-mimi
(``src/fast_mimi/config.py:29-294``): the same field names, defaults, derived
properties and JSON mapping, so ``config.json`` files written for one load in
the other.  Hub download is not part of this runtime; configs are read from a
local directory.
"""

from __future__ import annotations

import json
import math
from dataclasses import asdict, dataclass, fields
from pathlib import Path
from typing import Any

# Published identity of the kyutai/mimi checkpoint (config.py:18-26).
KYUTAI_MIMI_MODEL_ID = "kyutai/mimi"
KYUTAI_MIMI_REVISION = "89091b3e466eb6a9d11e537bf26b144f194978f7"
KYUTAI_MIMI_WEIGHTS_SHA256 = (
    "bac7e85083dcded655d24eaadde7e6eea34c0da1b35fa2d284e641bd2b942a5e"
)
KYUTAI_MIMI_PARAMETER_FINGERPRINT = (
    "3feaa6168b191ffdebfd8f695b963f72c8d847a3966f7cc3283af6b38d437bb4"
)
KYUTAI_MIMI_PARAMETER_COUNT = 79_308_609


@dataclass
class MimiConfig:
    """Architecture of the Mimi codec (defaults = published kyutai/mimi).

    SEANet: ``num_filters`` base width, ``upsampling_ratios`` decoder strides
    (the encoder walks them reversed), kernels ``kernel_size`` /
    ``residual_kernel_size`` / ``last_kernel_size``.  Transformers:
    ``num_hidden_layers`` pre-LN layers of width ``hidden_size`` with
    ``num_attention_heads`` heads of ``head_dim``, GELU FFN of
    ``intermediate_size``, causal window ``sliding_window`` and RoPE base
    ``rope_theta``.  RVQ: ``num_quantizers`` codebooks of ``codebook_size`` x
    ``codebook_dim``, the first ``num_semantic_quantizers`` forming the
    semantic branch.
    """

    sampling_rate: int = 24_000
    audio_channels: int = 1
    hidden_size: int = 512
    num_filters: int = 64
    num_residual_layers: int = 1
    upsampling_ratios: tuple[int, ...] = (8, 6, 5, 4)
    kernel_size: int = 7
    last_kernel_size: int = 3
    residual_kernel_size: int = 3
    dilation_growth_rate: int = 2
    use_causal_conv: bool = True
    pad_mode: str = "constant"
    compress: int = 2
    trim_right_ratio: float = 1.0

    codebook_size: int = 2048
    codebook_dim: int = 256
    num_quantizers: int = 32
    use_conv_shortcut: bool = False
    vector_quantization_hidden_dimension: int = 256
    num_semantic_quantizers: int = 1
    upsample_groups: int = 512

    num_hidden_layers: int = 8
    intermediate_size: int = 2048
    num_attention_heads: int = 8
    num_key_value_heads: int = 8
    head_dim: int | None = 64
    hidden_act: str = "gelu"
    max_position_embeddings: int = 8000
    initializer_range: float = 0.02
    norm_eps: float = 1e-5
    use_cache: bool = False
    use_streaming: bool = False
    rope_theta: float = 10_000.0
    sliding_window: int = 250
    attention_dropout: float = 0.0
    layer_scale_initial_scale: float = 0.01
    attention_bias: bool = False

    frame_rate_override: float | None = 12.5
    return_dict: bool = True

    def __post_init__(self) -> None:
        self.upsampling_ratios = tuple(int(r) for r in self.upsampling_ratios)
        if self.head_dim is None:
            self.head_dim = self.hidden_size // self.num_attention_heads
        if self.hidden_size % self.num_attention_heads:
            raise ValueError("hidden_size must be divisible by num_attention_heads")
        if self.num_attention_heads % self.num_key_value_heads:
            raise ValueError(
                "num_attention_heads must be divisible by num_key_value_heads"
            )
        if self.num_semantic_quantizers >= self.num_quantizers:
            raise ValueError(
                "num_semantic_quantizers must be smaller than num_quantizers"
            )
        if self.codebook_dim != self.vector_quantization_hidden_dimension:
            raise ValueError(
                "codebook_dim must match vector_quantization_hidden_dimension"
            )

    # Derived rates (config.py:155-192).
    @property
    def encodec_frame_rate(self) -> int:
        """SEANet output frames per second (before the 2x bottleneck)."""
        return math.ceil(self.sampling_rate / math.prod(self.upsampling_ratios))

    @property
    def frame_size(self) -> int:
        """Waveform samples per final code frame (all strides, incl. the 2x)."""
        return math.prod(self.upsampling_ratios) * 2

    @property
    def frame_rate(self) -> float:
        """Final code frames per second."""
        if self.frame_rate_override is not None:
            return self.frame_rate_override
        return self.sampling_rate / self.frame_size

    @property
    def num_codebooks(self) -> int:
        return self.num_quantizers

    # JSON mapping (config.py:194-294): ``frame_rate`` <-> ``frame_rate_override``.
    @classmethod
    def from_dict(cls, values: dict[str, Any]) -> "MimiConfig":
        known = {f.name for f in fields(cls)}
        mapped = dict(values)
        if "frame_rate" in mapped and "frame_rate_override" not in mapped:
            mapped["frame_rate_override"] = mapped.pop("frame_rate")
        return cls(**{k: v for k, v in mapped.items() if k in known})

    @classmethod
    def from_json_file(cls, path: str | Path) -> "MimiConfig":
        with Path(path).open(encoding="utf-8") as handle:
            return cls.from_dict(json.load(handle))

    @classmethod
    def from_pretrained(cls, model_id: str | Path, **_: Any) -> "MimiConfig":
        """Read ``config.json`` from a local checkpoint directory."""
        path = Path(model_id)
        if not path.is_dir():
            raise OSError(
                f"{model_id!r} is not a local directory; this runtime has no Hub access"
            )
        return cls.from_json_file(path / "config.json")

    def to_dict(self) -> dict[str, Any]:
        result = asdict(self)
        result["upsampling_ratios"] = list(self.upsampling_ratios)
        result["frame_rate"] = result.pop("frame_rate_override")
        return result

    def save_pretrained(self, directory: str | Path) -> Path:
        directory = Path(directory)
        directory.mkdir(parents=True, exist_ok=True)
        path = directory / "config.json"
        path.write_text(json.dumps(self.to_dict(), indent=2) + "\n", encoding="utf-8")
        return path
