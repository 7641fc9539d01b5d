"""Checkpoint layout and a portable seeded initialiser for Mimi.

``state_dict_spec`` lists every persistent tensor of the reference module tree
(kadirnar/fast-mimi ``src/fast_mimi/model.py``: encoder ``:1013-1049``,
transformers ``:2070-2090`` / ``:2000-2025`` / ``:1700-1760``, down/upsample
``:2730-2752``, decoder ``:1240-1286``, quantizer ``:2238-2480``) with its
checkpoint name, shape and initialiser, in ``state_dict()`` order.

``seeded_state_dict`` fills that layout without the torch global RNG: each
tensor draws from its own numpy PCG64 stream keyed by ``(seed, name)``, so the
weights are identical on every platform and independent of construction order.
Distributions follow ``MimiModel._initialize_weights`` (``model.py:2824-2850``):
Kaiming-normal convs (fan-in mode, gain sqrt(2)), uniform conv biases with bound
sqrt(groups / (in_channels * kernel)), N(0, initializer_range) linears, unit
LayerNorm, constant LayerScale; codebooks use embed_sum ~ N(0,1)/16 with unit
cluster usage (no checkpoint is available offline).
"""

from __future__ import annotations

import hashlib
import math
from dataclasses import dataclass

import numpy as np

from .config import MimiConfig


@dataclass(frozen=True)
class TensorSpec:
    name: str
    shape: tuple[int, ...]
    init: str  # conv_w | convt_w | conv_b | linear_w | ones | zeros | const | codebook
    fan_in: int = 0
    bound: float = 0.0
    value: float = 0.0


def _conv(specs, prefix, cin, cout, k, groups=1, bias=True):
    specs.append(TensorSpec(f"{prefix}.conv.weight", (cout, cin // groups, k),
                            "conv_w", fan_in=(cin // groups) * k))
    if bias:
        specs.append(TensorSpec(f"{prefix}.conv.bias", (cout,), "conv_b",
                                bound=math.sqrt(groups / (cin * k))))


def _convt(specs, prefix, cin, cout, k, groups=1, bias=True):
    # torch's fan-in of a ConvTranspose weight [in, out/g, k] is (out/g) * k.
    specs.append(TensorSpec(f"{prefix}.conv.weight", (cin, cout // groups, k),
                            "convt_w", fan_in=(cout // groups) * k))
    if bias:
        specs.append(TensorSpec(f"{prefix}.conv.bias", (cout,), "conv_b",
                                bound=math.sqrt(groups / (cin * k))))


def _resblock(specs, prefix, config, dim):
    hidden = dim // config.compress
    _conv(specs, f"{prefix}.block.1", dim, hidden, config.residual_kernel_size)
    _conv(specs, f"{prefix}.block.3", hidden, dim, 1)
    if config.use_conv_shortcut:
        _conv(specs, f"{prefix}.shortcut", dim, dim, 1)


def _transformer(specs, prefix, config):
    h = config.hidden_size
    hd = config.head_dim
    for i in range(config.num_hidden_layers):
        p = f"{prefix}.layers.{i}"
        for proj, out in (("q", config.num_attention_heads * hd),
                          ("k", config.num_key_value_heads * hd),
                          ("v", config.num_key_value_heads * hd)):
            specs.append(TensorSpec(f"{p}.self_attn.{proj}_proj.weight", (out, h), "linear_w"))
        specs.append(TensorSpec(f"{p}.self_attn.o_proj.weight",
                                (h, config.num_attention_heads * hd), "linear_w"))
        specs.append(TensorSpec(f"{p}.mlp.fc1.weight", (config.intermediate_size, h), "linear_w"))
        specs.append(TensorSpec(f"{p}.mlp.fc2.weight", (h, config.intermediate_size), "linear_w"))
        for ln in ("input_layernorm", "post_attention_layernorm"):
            specs.append(TensorSpec(f"{p}.{ln}.weight", (h,), "ones"))
            specs.append(TensorSpec(f"{p}.{ln}.bias", (h,), "zeros"))
        for ls in ("self_attn_layer_scale", "mlp_layer_scale"):
            specs.append(TensorSpec(f"{p}.{ls}.scale", (h,), "const",
                                    value=config.layer_scale_initial_scale))


def encoder_layer_indices(config: MimiConfig) -> dict[str, list[int]]:
    """Module indices of the encoder stack (``model.py:1013-1049``)."""
    idx = 1
    res, down = [], []
    for _ in reversed(config.upsampling_ratios):
        blocks = []
        for _r in range(config.num_residual_layers):
            blocks.append(idx)
            idx += 1
        res.append(blocks)
        idx += 1  # ELU
        down.append(idx)
        idx += 1
    idx += 1  # ELU
    return {"first": [0], "res": res, "down": down, "last": [idx]}


def decoder_layer_indices(config: MimiConfig) -> dict[str, list[int]]:
    """Module indices of the decoder stack (``model.py:1249-1286``)."""
    idx = 1
    up, res = [], []
    for _ in config.upsampling_ratios:
        idx += 1  # ELU
        up.append(idx)
        idx += 1
        blocks = []
        for _r in range(config.num_residual_layers):
            blocks.append(idx)
            idx += 1
        res.append(blocks)
    idx += 1  # ELU
    return {"first": [0], "up": up, "res": res, "last": [idx]}


def state_dict_spec(config: MimiConfig) -> list[TensorSpec]:
    specs: list[TensorSpec] = []
    nf = config.num_filters
    # Encoder.
    enc = encoder_layer_indices(config)
    _conv(specs, "encoder.layers.0", config.audio_channels, nf, config.kernel_size)
    scale = 1
    for stage, ratio in enumerate(reversed(config.upsampling_ratios)):
        ch = scale * nf
        for r, li in enumerate(enc["res"][stage]):
            _resblock(specs, f"encoder.layers.{li}", config, ch)
        _conv(specs, f"encoder.layers.{enc['down'][stage]}", ch, 2 * ch, 2 * ratio)
        scale *= 2
    _conv(specs, f"encoder.layers.{enc['last'][0]}", scale * nf, config.hidden_size,
          config.last_kernel_size)
    _transformer(specs, "encoder_transformer", config)
    if config.frame_rate != config.encodec_frame_rate:
        ratio = int(config.encodec_frame_rate / config.frame_rate)
        _conv(specs, "downsample", config.hidden_size, config.hidden_size, 2 * ratio,
              bias=False)
        _convt(specs, "upsample", config.hidden_size, config.hidden_size, 2 * ratio,
               groups=config.upsample_groups, bias=False)
    _transformer(specs, "decoder_transformer", config)
    # Decoder.
    dec = decoder_layer_indices(config)
    scale = 2 ** len(config.upsampling_ratios)
    _conv(specs, "decoder.layers.0", config.hidden_size, scale * nf, config.kernel_size)
    for stage, ratio in enumerate(config.upsampling_ratios):
        ch = scale * nf
        _convt(specs, f"decoder.layers.{dec['up'][stage]}", ch, ch // 2, 2 * ratio)
        for li in dec["res"][stage]:
            _resblock(specs, f"decoder.layers.{li}", config, ch // 2)
        scale //= 2
    _conv(specs, f"decoder.layers.{dec['last'][0]}", nf, config.audio_channels,
          config.last_kernel_size)
    # Quantizer.
    vq = config.vector_quantization_hidden_dimension
    branches = (("semantic", config.num_semantic_quantizers),
                ("acoustic", config.num_quantizers - config.num_semantic_quantizers))
    for branch, count in branches:
        p = f"quantizer.{branch}_residual_vector_quantizer"
        for j in range(count):
            cb = f"{p}.layers.{j}.codebook"
            specs.append(TensorSpec(f"{cb}.initialized", (1,), "ones"))
            specs.append(TensorSpec(f"{cb}.cluster_usage", (config.codebook_size,), "ones"))
            specs.append(TensorSpec(f"{cb}.embed_sum",
                                    (config.codebook_size, config.codebook_dim), "codebook"))
        if vq != config.hidden_size:
            specs.append(TensorSpec(f"{p}.input_proj.weight", (vq, config.hidden_size, 1),
                                    "conv_w", fan_in=config.hidden_size))
            specs.append(TensorSpec(f"{p}.output_proj.weight", (config.hidden_size, vq, 1),
                                    "conv_w", fan_in=vq))
    return specs


def _stream(seed: int, name: str) -> np.random.Generator:
    digest = hashlib.sha256(f"{seed}:{name}".encode()).digest()
    return np.random.Generator(np.random.PCG64(int.from_bytes(digest[:16], "little")))


def init_tensor(spec: TensorSpec, config: MimiConfig, seed: int) -> np.ndarray:
    rng = _stream(seed, spec.name)
    if spec.init in ("conv_w", "convt_w"):
        std = math.sqrt(2.0) / math.sqrt(spec.fan_in)
        out = rng.standard_normal(spec.shape) * std
    elif spec.init == "conv_b":
        out = rng.uniform(-spec.bound, spec.bound, spec.shape)
    elif spec.init == "linear_w":
        out = rng.standard_normal(spec.shape) * config.initializer_range
    elif spec.init == "ones":
        out = np.ones(spec.shape)
    elif spec.init == "zeros":
        out = np.zeros(spec.shape)
    elif spec.init == "const":
        out = np.full(spec.shape, spec.value)
    elif spec.init == "codebook":
        out = rng.standard_normal(spec.shape) / 16.0
    else:  # pragma: no cover - spec kinds are closed
        raise ValueError(spec.init)
    return np.ascontiguousarray(out, dtype=np.float32)


def seeded_state_dict(config: MimiConfig, seed: int = 0) -> dict[str, np.ndarray]:
    """Deterministic full state dict (numpy float32) for ``config``."""
    return {s.name: init_tensor(s, config, seed) for s in state_dict_spec(config)}


def parameter_count(config: MimiConfig) -> int:
    """Number of learnable parameters (codebook buffers excluded)."""
    n = 0
    for s in state_dict_spec(config):
        if ".codebook." in s.name:
            continue
        n += int(np.prod(s.shape))
    return n
