"""Streaming state: the convolution padding cache and the sliding KV cache.

Same constructors, attributes and methods as the reference's
``MimiConv1dPaddingCache`` (``model.py:521-620``) and ``MimiKVCache``
(``model.py:363-518``).  Storage is device-resident and channels-last to match
the HIP kernels:

* ``MimiConv1dPaddingCache.padding_cache[i]`` is ``[batch, padding, channels]``
  (the reference keeps ``[batch, channels, padding]``).  It holds the last
  ``padding`` rows of the layer's input.  For the first convolution of a
  residual block these are the rows *before* the block's ELU, which the kernel
  applies as it loads them; everywhere else they are the convolution input
  itself.
* ``MimiKVCache.key_cache[i]`` / ``value_cache[i]`` are
  ``[batch, frames, kv_heads * head_dim]`` of rotated keys / values (the
  reference keeps ``[batch, kv_heads, frames, head_dim]``).
"""

from __future__ import annotations

import torch


class MimiConv1dPaddingCache:
    """Per-layer left context for chunked causal convolution (``model.py:521-620``)."""

    def __init__(self, num_layers: int, per_layer_padding: list[int],
                 per_layer_padding_mode: list[str], per_layer_in_channels: list[int]) -> None:
        lengths = {len(per_layer_padding), len(per_layer_padding_mode), len(per_layer_in_channels)}
        if lengths != {num_layers}:
            raise ValueError("all per-layer cache settings must contain num_layers entries")
        for mode in per_layer_padding_mode:
            if mode not in ("constant", "replicate"):
                raise NotImplementedError(f"padding mode {mode!r} is not supported for streaming")
        self.per_layer_padding = list(per_layer_padding)
        self.per_layer_padding_mode = list(per_layer_padding_mode)
        self.per_layer_in_channels = list(per_layer_in_channels)
        self.padding_cache: list[torch.Tensor | None] = [None] * num_layers

    def update(self, hidden_states: torch.Tensor, layer_idx: int) -> torch.Tensor:
        """Advance one layer: return its prior context ``[B, padding, C]`` and
        keep the newest ``padding`` rows of context + ``hidden_states``
        (channels-last ``[B, L, C]``)."""
        pad = self.per_layer_padding[layer_idx]
        current = self.padding_cache[layer_idx]
        if current is None:
            b, _, c = hidden_states.shape
            if self.per_layer_padding_mode[layer_idx] == "constant":
                current = hidden_states.new_zeros((b, pad, c))
            else:
                current = hidden_states[:, :1].expand(b, pad, c).contiguous()
        if pad > 0:
            joined = torch.cat((current, hidden_states), dim=1)
            self.padding_cache[layer_idx] = joined[:, joined.shape[1] - pad:].contiguous()
        else:
            self.padding_cache[layer_idx] = hidden_states[:, :0].contiguous()
        return current


class MimiKVCache:
    """Sliding-window key/value cache with unbounded position count (``model.py:363-518``)."""

    def __init__(self, num_layers: int = 0, sliding_window: int | None = None) -> None:
        if sliding_window is not None and sliding_window <= 0:
            raise ValueError("sliding_window must be positive")
        self.sliding_window = sliding_window
        self.key_cache: list[torch.Tensor | None] = [None] * num_layers
        self.value_cache: list[torch.Tensor | None] = [None] * num_layers
        self._cumulative_lengths: list[int] = [0] * num_layers

    def _ensure_layer(self, layer_idx: int) -> None:
        missing = layer_idx + 1 - len(self.key_cache)
        if missing > 0:
            self.key_cache.extend([None] * missing)
            self.value_cache.extend([None] * missing)
            self._cumulative_lengths.extend([0] * missing)

    def _retained(self, t: torch.Tensor) -> torch.Tensor:
        if self.sliding_window is None:
            return t
        keep = self.sliding_window - 1
        return t[:, :0].contiguous() if keep == 0 else t[:, -keep:].contiguous()

    def configure_sliding_window(self, sliding_window: int) -> None:
        """Set the window (or check it matches) and crop stored frames to ``window - 1``."""
        if sliding_window <= 0:
            raise ValueError("sliding_window must be positive")
        if self.sliding_window is not None:
            if self.sliding_window != sliding_window:
                raise ValueError("cache sliding_window does not match the model configuration")
            return
        self.sliding_window = sliding_window
        for i, key in enumerate(self.key_cache):
            if key is None:
                continue
            if self._cumulative_lengths[i] == 0:
                self._cumulative_lengths[i] = key.shape[1]
            self.key_cache[i] = self._retained(key)
            self.value_cache[i] = self._retained(self.value_cache[i])

    def update(self, key: torch.Tensor, value: torch.Tensor, layer_idx: int):
        """Append ``[B, frames, kv_dim]`` keys/values; return everything visible
        to this step (stored frames followed by the new ones)."""
        self._ensure_layer(layer_idx)
        self._cumulative_lengths[layer_idx] += key.shape[1]
        if self.key_cache[layer_idx] is not None:
            key = torch.cat((self.key_cache[layer_idx], key), dim=1)
            value = torch.cat((self.value_cache[layer_idx], value), dim=1)
        self.key_cache[layer_idx] = self._retained(key)
        self.value_cache[layer_idx] = self._retained(value)
        return key, value

    def get_seq_length(self, layer_idx: int = 0) -> int:
        """Frames ever appended to the layer (including cropped ones)."""
        if layer_idx >= len(self._cumulative_lengths):
            return 0
        return self._cumulative_lengths[layer_idx]

    def get_mask_sizes(self, query_length: int, layer_idx: int = 0) -> tuple[int, int]:
        """``(key_length, key_offset)`` of the keys an upcoming query chunk sees."""
        cumulative = self.get_seq_length(layer_idx)
        if self.sliding_window is None:
            return cumulative + query_length, 0
        key_offset = max(cumulative - self.sliding_window + 1, 0)
        if cumulative >= self.sliding_window:
            return self.sliding_window - 1 + query_length, key_offset
        return cumulative + query_length, key_offset

    def to(self, device) -> "MimiKVCache":
        self.key_cache = [t.to(device) if t is not None else None for t in self.key_cache]
        self.value_cache = [t.to(device) if t is not None else None for t in self.value_cache]
        return self
