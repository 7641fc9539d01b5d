"""``MimiModel``: the fast-mimi public surface on the MI355X runtime.

Mirrors kadirnar/fast-mimi ``src/fast_mimi/model.py``: ``from_pretrained``
(``:2852-2941``), ``save_pretrained`` (``:2943-2962``), ``encode``
(``:3070-3137``), ``decode`` (``:3172-3202``), ``forward`` (``:3452-3538``),
``get_encoded_length`` (``:3007-3024``), ``get_audio_codes_mask``
(``:3026-3045``) and the ``MimiOutput`` family (``:168-262``), with the same
argument meaning, validation errors and output ownership (returned tensors are
fresh, caller-owned).

Differences, by design:
  * execution is the HIP library on a ROCm GPU; there is no CPU or eager
    fallback — a model on the CPU can be built, saved and loaded, but running
    it raises ``RuntimeError``;
  * ``MimiModel(config)`` initialises from a portable seeded generator
    (``weights.seeded_state_dict``) instead of the torch global RNG;
  * a Hub model id resolves only through an existing local Hugging Face cache
    (``cache_dir`` / ``local_files_only``); nothing is downloaded;
  * stateful calls (``encoder_past_key_values``, ``padding_cache``,
    ``use_streaming``, ``decoder_past_key_values``) run eagerly, since their
    cache lengths change from call to call; every other call replays a
    captured hipGraph per input shape.
"""

from __future__ import annotations

import hashlib
import threading
from dataclasses import dataclass, fields
from pathlib import Path
from typing import Any, Iterator

import numpy as np
import torch

from .config import (
    KYUTAI_MIMI_MODEL_ID,
    KYUTAI_MIMI_PARAMETER_COUNT,
    KYUTAI_MIMI_REVISION,
    KYUTAI_MIMI_WEIGHTS_SHA256,
    MimiConfig,
)
from . import _native as nat
from .streaming import MimiConv1dPaddingCache, MimiKVCache
from .weights import encoder_layer_indices, seeded_state_dict, state_dict_spec


class _OutputMixin:
    """Tuple / mapping access of ``ModelOutput`` (``model.py:168-231``):
    ``None`` fields are skipped positionally, names always resolve."""

    def _present(self) -> tuple[Any, ...]:
        return tuple(getattr(self, f.name) for f in fields(self) if getattr(self, f.name) is not None)

    def __getitem__(self, key):
        if isinstance(key, str):
            return getattr(self, key)
        return self._present()[key]

    def __iter__(self) -> Iterator[Any]:
        return iter(self._present())

    def __len__(self) -> int:
        return len(self._present())

    def get(self, key: str, default: Any = None) -> Any:
        return getattr(self, key, default)


@dataclass
class MimiOutput(_OutputMixin):
    audio_codes: torch.Tensor | None = None
    audio_values: torch.Tensor | None = None
    encoder_past_key_values: Any = None
    decoder_past_key_values: Any = None


@dataclass
class MimiEncoderOutput(_OutputMixin):
    audio_codes: torch.Tensor | None = None
    encoder_past_key_values: Any = None
    padding_cache: Any = None


@dataclass
class MimiDecoderOutput(_OutputMixin):
    audio_values: torch.Tensor | None = None
    decoder_past_key_values: Any = None


# Architecture fields the declared checkpoint must keep (``model.py:76-81``).
DECLARED_MIMI_CONFIG = {"sampling_rate": 24_000, "frame_rate": 12.5, "audio_channels": 1,
                        "codebook_size": 2_048}


def assert_declared_mimi_config(config: MimiConfig) -> None:
    """Reject architecture drift of the identity-locked checkpoint
    (``_assert_declared_mimi_config``, ``model.py:92-100``)."""
    for name, expected in DECLARED_MIMI_CONFIG.items():
        actual = getattr(config, name)
        if actual != expected:
            raise RuntimeError(f"declared checkpoint config {name!r} changed: {actual!r} != {expected!r}")


def _file_sha256(path: Path) -> str:
    digest = hashlib.sha256()
    with path.open("rb") as handle:
        for block in iter(lambda: handle.read(1 << 20), b""):
            digest.update(block)
    return digest.hexdigest()


class _GraphRunner:
    """One captured hipGraph of a fixed-shape call with static input buffers
    (the role of ``_MimiCudaGraphRunner``, ``model.py:281-343``)."""

    def __init__(self, fn, inputs: tuple[torch.Tensor, ...], device):
        self.device = device
        self.static_in = tuple(t.clone() for t in inputs)
        self.lock = threading.Lock()
        side = torch.cuda.Stream(device)
        side.wait_stream(torch.cuda.current_stream(device))
        with torch.cuda.stream(side):
            fn(*self.static_in)  # warm-up outside capture
        torch.cuda.current_stream(device).wait_stream(side)
        self.graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(self.graph):
            self.static_out = fn(*self.static_in)

    def __call__(self, *inputs: torch.Tensor):
        with self.lock:
            _copy_pairs(list(zip(inputs, self.static_in)), self.device)
            self.graph.replay()
            # Caller-owned copies of the outputs, so a later replay cannot
            # change what this call returned.
            outs = self.static_out if isinstance(self.static_out, tuple) else (self.static_out,)
            fresh = tuple(torch.empty_like(t) for t in outs)
            _copy_pairs(list(zip(outs, fresh)), self.device)
            return fresh if isinstance(self.static_out, tuple) else fresh[0]


def _copy_pairs(pairs, device) -> None:
    """dst <- src for each (src, dst) pair, two pairs per fm_copy_buffers
    launch (one launch where torch would issue one copy per tensor); pairs
    that are not same-dtype, same-shape contiguous tensors go through
    ``Tensor.copy_``."""
    plain = []
    for src, dst in pairs:
        if (src.dtype == dst.dtype and src.shape == dst.shape and src.is_contiguous()
                and dst.is_contiguous() and src.device == dst.device):
            plain.append((src, dst))
        else:
            dst.copy_(src)
    stream = torch.cuda.current_stream(device).cuda_stream
    for i in range(0, len(plain), 2):
        (s0, d0), (s1, d1) = plain[i], plain[i + 1] if i + 1 < len(plain) else (None, None)
        nat.call("fm_copy_buffers", s0.data_ptr(), d0.data_ptr(), s0.numel() * s0.element_size(),
                 None if s1 is None else s1.data_ptr(), None if d1 is None else d1.data_ptr(),
                 0 if s1 is None else s1.numel() * s1.element_size(), stream)


class MimiModel:
    """Mimi neural audio codec on one MI355X GPU."""

    def __init__(self, config: MimiConfig | None = None, *, attention_backend: str = "sdpa",
                 device: torch.device | str | None = None, seed: int = 0,
                 use_graphs: bool = True) -> None:
        if attention_backend not in {"sdpa", "eager"}:
            raise ValueError("attention_backend must be 'sdpa' or 'eager'")
        self.config = MimiConfig() if config is None else config
        self.attention_backend = attention_backend
        self.bits_per_codebook = int(np.log2(self.config.codebook_size))
        if 2 ** self.bits_per_codebook != self.config.codebook_size:
            raise ValueError("codebook_size must be a power of two")
        self._spec = state_dict_spec(self.config)
        self._state = {k: torch.from_numpy(v) for k, v in seeded_state_dict(self.config, seed).items()}
        self.device = torch.device("cpu")
        self.use_graphs = use_graphs
        self._runtime = None
        self._graphs: dict[tuple, _GraphRunner] = {}
        self.training = False
        if device is not None:
            self.to(device)

    # ------------------------------------------------------------ state
    def state_dict(self) -> dict[str, torch.Tensor]:
        return dict(self._state)

    def load_state_dict(self, state: dict[str, torch.Tensor], strict: bool = True):
        expected = {s.name: s.shape for s in self._spec}
        missing = [k for k in expected if k not in state]
        unexpected = [k for k in state if k not in expected]
        if strict and (missing or unexpected):
            raise RuntimeError(f"state_dict mismatch: missing={missing[:5]} unexpected={unexpected[:5]}")
        for k, shape in expected.items():
            if k in state and tuple(state[k].shape) != tuple(shape):
                raise RuntimeError(f"size mismatch for {k}: {tuple(state[k].shape)} != {shape}")
        for k in expected:
            if k in state:
                self._state[k] = state[k].detach().to(device=self.device, dtype=torch.float32).clone()
        self._invalidate()
        return missing, unexpected

    def parameters(self) -> Iterator[torch.Tensor]:
        for s in self._spec:
            if ".codebook." not in s.name:
                yield self._state[s.name]

    def release_graphs(self) -> None:
        """Drop every captured hipGraph (and the device memory its pool holds)."""
        self._graphs.clear()
        if torch.cuda.is_available():
            torch.cuda.empty_cache()

    def _invalidate(self) -> None:
        self._runtime = None
        self._graphs.clear()

    def to(self, device=None, dtype=None) -> "MimiModel":
        if dtype is not None and dtype != torch.float32:
            raise ValueError("fast_mimi_amd computes in float32 only")
        if device is not None:
            device = torch.device(device)
            if device.type == "cuda" and device.index is None:
                device = torch.device("cuda", torch.cuda.current_device())
            self._state = {k: v.to(device) for k, v in self._state.items()}
            self.device = device
            self._invalidate()
        return self

    def cuda(self, device=None) -> "MimiModel":
        return self.to(torch.device("cuda") if device is None else device)

    def eval(self) -> "MimiModel":
        return self

    def __call__(self, *args, **kwargs):
        return self.forward(*args, **kwargs)

    # ------------------------------------------------------- checkpoint I/O
    @classmethod
    def from_pretrained(cls, model_id: str | Path = KYUTAI_MIMI_MODEL_ID, *,
                        revision: str = KYUTAI_MIMI_REVISION, cache_dir=None,
                        local_files_only: bool = False, attention_backend: str = "sdpa",
                        device=None, dtype=None) -> "MimiModel":
        """Load ``config.json`` + ``model.safetensors`` strictly
        (``model.py:2852-2941``).

        ``model_id`` is a local directory, or a Hub repository id resolved by
        ``huggingface_hub.hf_hub_download(..., revision, cache_dir,
        local_files_only)`` exactly as the reference does (``:2898-2920``); with
        ``local_files_only=True`` that reads an existing cache and never touches
        the network.  The declared ``kyutai/mimi`` checkpoint keeps the
        reference's identity locks, in its order: revision, declared config
        fields (``_assert_declared_mimi_config``, ``:92-100``), weights SHA-256,
        parameter count."""
        from safetensors.torch import load_file

        declared = str(model_id) == KYUTAI_MIMI_MODEL_ID
        if declared and revision != KYUTAI_MIMI_REVISION:
            raise ValueError(
                f"declared kyutai/mimi revision changed: {revision!r} != {KYUTAI_MIMI_REVISION!r}")
        path = Path(model_id)
        if path.exists():
            config_path, weights = path / "config.json", path / "model.safetensors"
        else:
            from huggingface_hub import hf_hub_download

            config_path, weights = (
                Path(hf_hub_download(str(model_id), name, revision=revision, cache_dir=cache_dir,
                                     local_files_only=local_files_only))
                for name in ("config.json", "model.safetensors"))
        config = MimiConfig.from_json_file(config_path)
        if declared:
            assert_declared_mimi_config(config)
            digest = _file_sha256(weights)
            if digest != KYUTAI_MIMI_WEIGHTS_SHA256:
                raise RuntimeError(
                    f"declared kyutai/mimi checkpoint digest changed: {digest} != {KYUTAI_MIMI_WEIGHTS_SHA256}")
        model = cls(config, attention_backend=attention_backend)
        model.load_state_dict(load_file(str(weights), device="cpu"), strict=True)
        if declared:
            count = sum(p.numel() for p in model.parameters())
            if count != KYUTAI_MIMI_PARAMETER_COUNT:
                raise RuntimeError(
                    f"declared kyutai/mimi parameter count changed: {count} != {KYUTAI_MIMI_PARAMETER_COUNT}")
        if device is not None or dtype is not None:
            model.to(device=device, dtype=dtype)
        return model.eval()

    def save_pretrained(self, directory: str | Path) -> None:
        from safetensors.torch import save_file

        directory = Path(directory)
        directory.mkdir(parents=True, exist_ok=True)
        self.config.save_pretrained(directory)
        state = {k: v.detach().cpu().contiguous() for k, v in self._state.items()}
        save_file(state, str(directory / "model.safetensors"), metadata={"format": "pt"})

    # ------------------------------------------------------------ runtime
    def runtime(self):
        if self.device.type != "cuda":
            raise RuntimeError("fast_mimi_amd executes on a ROCm GPU; move the model with .to('cuda')")
        if self._runtime is None:
            from .runtime import MimiRuntime

            with torch.cuda.device(self.device):
                self._runtime = MimiRuntime(self.config, self._state, self.device)
        return self._runtime

    def _check_audio(self, input_values: torch.Tensor) -> None:
        if input_values.ndim != 3:
            raise ValueError("input_values must have shape [batch, channels, samples]")
        if not 1 <= input_values.shape[1] <= 2:
            raise ValueError("input audio must have one or two channels")
        if input_values.shape[1] != self.config.audio_channels:
            raise ValueError(
                f"expected {self.config.audio_channels} audio channel(s), got {input_values.shape[1]}")

    def _resolve_count(self, num_quantizers: int | None) -> int:
        count = self.config.num_quantizers if num_quantizers is None else int(num_quantizers)
        if count > self.config.num_quantizers:
            raise ValueError(f"num_quantizers must be <= {self.config.num_quantizers}, got {count}")
        if count < self.config.num_semantic_quantizers:
            raise ValueError(
                f"num_quantizers must be >= {self.config.num_semantic_quantizers}, got {count}")
        return count

    def _on_device(self, t: torch.Tensor, dtype) -> torch.Tensor:
        if t.device != self.device:
            raise ValueError(f"tensor on {t.device}, model on {self.device}")
        return t.to(dtype).contiguous()

    def _graph(self, key, fn, inputs):
        runner = self._graphs.get(key)
        if runner is None:
            runner = _GraphRunner(fn, inputs, self.device)
            self._graphs[key] = runner
        return runner(*inputs)

    def _prepare_lengths(self, samples: int) -> None:
        rt = self.runtime()
        t25 = self._frames_25(samples)
        rt.prepare(t25)

    def _frames_25(self, samples: int) -> int:
        n = samples
        for r in reversed(self.config.upsampling_ratios):
            n = -(-n // r)
        return n

    # ------------------------------------------------------------ public API
    def encode(self, input_values: torch.Tensor, padding_mask: torch.Tensor | None = None,
               num_quantizers: int | None = None, encoder_past_key_values=None,
               padding_cache=None, use_streaming: bool | None = None,
               return_dict: bool | None = None):
        """Encode ``[B, C, S]`` audio to int64 codes ``[B, nq, T]``.  The padding
        mask does not change encoding (``model.py:3123-3134``)."""
        return_dict = self.config.return_dict if return_dict is None else return_dict
        use_streaming = self.config.use_streaming if use_streaming is None else use_streaming
        count = self._resolve_count(num_quantizers)
        self._check_audio(input_values)
        rt = self.runtime()
        audio = self._on_device(input_values, torch.float32)
        if use_streaming and padding_cache is None:
            padding_cache = self._new_padding_cache()
        if use_streaming and encoder_past_key_values is None:
            encoder_past_key_values = MimiKVCache(self.config.num_hidden_layers, self.config.sliding_window)
        if padding_cache is not None or encoder_past_key_values is not None:
            # Stateful calls run eagerly: cache lengths change from call to call.
            with torch.cuda.device(self.device), torch.inference_mode():
                codes = rt.encode(audio, count, padding_cache, encoder_past_key_values)
            if not return_dict:
                return codes, encoder_past_key_values, padding_cache
            return MimiEncoderOutput(codes, encoder_past_key_values, padding_cache)
        self._prepare_lengths(audio.shape[-1])
        with torch.cuda.device(self.device), torch.inference_mode():
            if self.use_graphs:
                codes = self._graph(("enc", tuple(audio.shape), count),
                                    lambda a: rt.encode(a, count), (audio,))
            else:
                codes = rt.encode(audio, count)
        if not return_dict:
            return codes, None, None
        return MimiEncoderOutput(codes, None, None)

    def decode(self, audio_codes: torch.Tensor, padding_mask: torch.Tensor | None = None,
               decoder_past_key_values=None, return_dict: bool | None = None):
        """Decode int64 codes ``[B, nq, T]`` to audio ``[B, C, T * frame_size]``,
        cropped to ``padding_mask.shape[-1]`` when that is shorter."""
        return_dict = self.config.return_dict if return_dict is None else return_dict
        if audio_codes.ndim != 3:
            raise ValueError("audio_codes must have shape [batch, codebooks, frames]")
        if not 1 <= audio_codes.shape[1] <= self.config.num_quantizers:
            raise ValueError(f"audio_codes must hold 1..{self.config.num_quantizers} codebooks")
        rt = self.runtime()
        codes = self._on_device(audio_codes, torch.int64)
        if codes.numel():
            lo, hi = torch.aminmax(codes)
            lo, hi = torch.stack((lo, hi)).tolist()  # one device->host sync
            if lo < 0 or hi >= self.config.codebook_size:
                raise IndexError("audio code out of range of the codebook")
        out_len = None if padding_mask is None else padding_mask.shape[-1]
        frames = codes.shape[-1]
        kv = decoder_past_key_values
        with torch.cuda.device(self.device), torch.inference_mode():
            if kv is not None:
                audio = rt.decode(codes, out_len, kv)
            elif self.use_graphs:
                rt.prepare(frames * (2 if rt.bottleneck else 1))
                audio = self._graph(("dec", tuple(codes.shape), out_len),
                                    lambda c: rt.decode(c, out_len), (codes,))
            else:
                rt.prepare(frames * (2 if rt.bottleneck else 1))
                audio = rt.decode(codes, out_len)
        if not return_dict:
            return audio, kv
        return MimiDecoderOutput(audio, kv)

    def forward(self, input_values: torch.Tensor, padding_mask: torch.Tensor | None = None,
                num_quantizers: int | None = None, audio_codes: torch.Tensor | None = None,
                encoder_past_key_values=None, decoder_past_key_values=None,
                return_dict: bool | None = None):
        """Encode→decode round trip (``model.py:3452-3538``); with ``audio_codes``
        given, decode only.  The mask crops the decoded audio to its length."""
        return_dict = self.config.return_dict if return_dict is None else return_dict
        mask = padding_mask
        if audio_codes is not None or encoder_past_key_values is not None or decoder_past_key_values is not None:
            # Decode-only, or stateful: the encode/decode entry points, eagerly where a cache is given.
            if mask is None:
                mask = torch.ones_like(input_values, dtype=torch.bool)
            if audio_codes is None:
                enc = self.encode(input_values, mask, num_quantizers, encoder_past_key_values,
                                  return_dict=True)
                audio_codes, encoder_past_key_values = enc.audio_codes, enc.encoder_past_key_values
            dec = self.decode(audio_codes, mask, decoder_past_key_values, return_dict=True)
            codes, audio = audio_codes, dec.audio_values
            decoder_past_key_values = dec.decoder_past_key_values
        else:
            count = self._resolve_count(num_quantizers)
            self._check_audio(input_values)
            rt = self.runtime()
            audio_in = self._on_device(input_values, torch.float32)
            out_len = input_values.shape[-1] if mask is None else mask.shape[-1]
            self._prepare_lengths(audio_in.shape[-1])

            def roundtrip(a):
                c = rt.encode(a, count)
                return c, rt.decode(c, out_len)

            with torch.cuda.device(self.device), torch.inference_mode():
                if self.use_graphs:
                    codes, audio = self._graph(("fwd", tuple(audio_in.shape), count, out_len),
                                               roundtrip, (audio_in,))
                else:
                    codes, audio = roundtrip(audio_in)
        if not return_dict:
            return codes, audio, encoder_past_key_values, decoder_past_key_values
        return MimiOutput(codes, audio, encoder_past_key_values, decoder_past_key_values)

    def _new_padding_cache(self) -> MimiConv1dPaddingCache:
        """Empty streaming conv cache over the encoder convolutions and the
        bottleneck downsample, in module order (``model.py:3047-3068``)."""
        layers = self.runtime().stream_conv_layers()
        return MimiConv1dPaddingCache(
            len(layers), [c.k - c.stride for c, _ in layers], [m for _, m in layers],
            [c.c_in for c, _ in layers])

    # -------------------------------------------------------- length helpers
    def get_encoded_length(self, input_length: torch.Tensor) -> torch.Tensor:
        """Waveform samples -> code frames (``model.py:3007-3024``): every causal
        conv maps L to ceil(L / stride); the bottleneck halves again."""
        n = torch.as_tensor(input_length, dtype=torch.int64)
        for r in reversed(self.config.upsampling_ratios):
            n = torch.div(n + r - 1, r, rounding_mode="floor")
        if self.config.frame_rate != self.config.encodec_frame_rate:
            n = torch.div(n + 1, 2, rounding_mode="floor")
        return n

    def get_audio_codes_mask(self, padding_mask: torch.Tensor, padding_side: str = "right") -> torch.Tensor:
        """Sample mask -> frame mask (``model.py:3026-3045``), with the
        reference's broadcasting: a 2-D ``[B, S]`` mask gives ``[B, T]``; a
        3-D ``[B, C, S]`` mask gives ``[B, B, T]`` (the per-row lengths
        ``[B, C]`` gain a trailing axis and broadcast against ``[B, T]``)."""
        lengths = self.get_encoded_length(padding_mask.sum(dim=-1))
        mask = torch.arange(int(lengths.max()), device=lengths.device).expand(len(lengths), -1)
        mask = mask < lengths.unsqueeze(1)
        return mask if padding_side == "right" else mask.flip(-1)
