"""CPU oracle for the Mimi encode/decode hot path — TEST INFRASTRUCTURE ONLY.

This module is the checker, never the product: only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The shipped path (``fast_mimi_amd``) runs on the HIP library and fails
loudly without it.

It restates, in PyTorch eager on the CPU and for any batch size, the portable
path of kadirnar/fast-mimi (``src/fast_mimi/model.py``), op for op and in the
same order, so that on the same machine its outputs equal the reference's bit
for bit.  Each function names the reference lines it follows.

Pins (see ``tests/test_oracle.py``):
  * reference golden vectors (``tests/golden/*.npz``, written by
    ``tests/golden/make_golden.py`` from the reference itself): codes and
    waveforms, tiny and full-size configs — bit-exact;
  * Hugging Face ``transformers.MimiModel`` at the reference's tiny test config
    (the reference's own test oracle, ``tests/conftest.py:31-55``) — bit-exact,
    offline and streaming (padding-cache encode, KV-cache decode; also the
    full config's streaming encode);
  * float64 brute force of every primitive on tiny inputs (conv padding and
    stride alignment, transposed-conv trim, replicate padding, RoPE, windowed
    causal softmax attention, LayerNorm, exact-erf GELU, ELU, the cdist
    mm-form, lowest-index argmin, RVQ decode add order);
  * closed-form encoded lengths (``tests/test_config.py:45-48`` of the
    reference).
"""

from __future__ import annotations

import math
from dataclasses import dataclass, field

import torch
import torch.nn.functional as F


# --------------------------------------------------------------------------
# Convolution primitives (model.py:697-797, :886-897).
# --------------------------------------------------------------------------

def causal_conv1d(x, weight, bias, stride=1, dilation=1, groups=1, pad_mode="constant"):
    """``MimiConv1d.forward`` offline branch (model.py:697-797).

    Left pad = effective_kernel - stride; right pad = (-L) mod stride (the
    stride-alignment 'extra' of ``_get_extra_padding_for_conv1d``, :697-707);
    the pad happens with ``pad_mode`` before the unpadded ``conv1d``.
    """
    k_eff = (weight.shape[-1] - 1) * dilation + 1
    left = k_eff - stride
    extra = (-x.shape[-1]) % stride
    if pad_mode == "constant":
        x = F.pad(x, (left, extra), "constant", 0.0)
    else:
        x = F.pad(x, (left, extra), pad_mode)
    return F.conv1d(x, weight, bias, stride, 0, dilation, groups)


def causal_conv_transpose1d(x, weight, bias, stride, groups=1):
    """``MimiConvTranspose1d.forward`` (model.py:886-897), trim ratio 1.0.

    All ``kernel - stride`` surplus samples are trimmed on the right.
    """
    y = F.conv_transpose1d(x, weight, bias, stride, 0, 0, groups)
    trim = weight.shape[-1] - stride
    return y[..., 0: y.shape[-1] - trim]


def elu(x):
    """``nn.ELU()`` (alpha 1) as used between SEANet layers."""
    return F.elu(x)


def conv_output_length(length, kernel, stride, dilation=1):
    """Closed form of ``MimiConv1d._get_output_length`` (model.py:734-761)."""
    k_eff = (kernel - 1) * dilation + 1
    pad_total = k_eff - stride
    frames = math.ceil((length - k_eff + pad_total) / stride + 1) - 1
    ideal = frames * stride + k_eff - pad_total
    extra = ideal - length
    total = length + pad_total + extra
    return (total - dilation * (kernel - 1) - 1) // stride + 1


# --------------------------------------------------------------------------
# Model
# --------------------------------------------------------------------------

@dataclass
class Trace:
    """Intermediates kept for diagnostics (near-tie margins, stage checks)."""
    encoder_out: torch.Tensor | None = None
    transformer_out: torch.Tensor | None = None
    downsampled: torch.Tensor | None = None
    rvq_inputs: list = field(default_factory=list)  # per codebook: [N, D] query rows
    quantized: torch.Tensor | None = None
    decoder_in: torch.Tensor | None = None


class KVState:
    """Per-layer retained rotated keys/values ``[B, H, n, D]`` plus the
    cumulative position count (``MimiKVCache``, model.py:363-518)."""

    def __init__(self, layers):
        self.keys = [None] * layers
        self.values = [None] * layers
        self.length = 0


@dataclass
class StreamState:
    """Encoder streaming state: per-conv left contexts (keyed by module
    prefix) and the encoder transformer's KV cache."""
    encoder_kv: KVState
    conv: dict = field(default_factory=dict)


class MimiOracle:
    """Batch-general restatement of ``MimiModel`` (model.py:2702-3538)."""

    def __init__(self, config, state: dict[str, torch.Tensor]):
        self.config = config
        self.state = {k: v.detach().to("cpu", torch.float32).contiguous() for k, v in state.items()}
        self._embeds: dict[str, torch.Tensor] = {}
        self.enc_res, self.enc_down, self.enc_last = self._enc_indices()
        self.dec_up, self.dec_res, self.dec_last = self._dec_indices()

    # Module indices of the SEANet stacks (model.py:1013-1049, :1249-1286).
    def _enc_indices(self):
        idx, res, down = 1, [], []
        for _ in reversed(self.config.upsampling_ratios):
            res.append(list(range(idx, idx + self.config.num_residual_layers)))
            idx += self.config.num_residual_layers + 1
            down.append(idx)
            idx += 1
        return res, down, idx + 1

    def _dec_indices(self):
        idx, up, res = 1, [], []
        for _ in self.config.upsampling_ratios:
            up.append(idx + 1)
            idx += 2
            res.append(list(range(idx, idx + self.config.num_residual_layers)))
            idx += self.config.num_residual_layers
        return up, res, idx + 1

    def _w(self, name):
        return self.state[name]

    def _conv(self, x, prefix, stride=1, dilation=1, pad_mode="constant", groups=1):
        return causal_conv1d(x, self._w(f"{prefix}.conv.weight"),
                             self.state.get(f"{prefix}.conv.bias"),
                             stride, dilation, groups, pad_mode)

    def _convt(self, x, prefix, stride, groups=1):
        return causal_conv_transpose1d(x, self._w(f"{prefix}.conv.weight"),
                                       self.state.get(f"{prefix}.conv.bias"),
                                       stride, groups)

    def _resblock(self, x, prefix, dilation):
        """``MimiResnetBlock.forward`` (model.py:947-971): x + conv1x1(ELU(conv_k(ELU(x))))."""
        h = elu(x)
        h = self._conv(h, f"{prefix}.block.1", dilation=dilation)
        h = elu(h)
        h = self._conv(h, f"{prefix}.block.3")
        residual = x
        if self.config.use_conv_shortcut:
            residual = self._conv(x, f"{prefix}.shortcut")
        return residual + h

    def encoder(self, x):
        """``MimiEncoder._forward_eager`` (model.py:1067-1084)."""
        cfg = self.config
        h = self._conv(x, "encoder.layers.0")
        for stage, ratio in enumerate(reversed(cfg.upsampling_ratios)):
            for r, li in enumerate(self.enc_res[stage]):
                h = self._resblock(h, f"encoder.layers.{li}", cfg.dilation_growth_rate ** r)
            h = elu(h)
            h = self._conv(h, f"encoder.layers.{self.enc_down[stage]}", stride=ratio)
        h = elu(h)
        return self._conv(h, f"encoder.layers.{self.enc_last}")

    def decoder(self, x):
        """``MimiDecoder._forward_eager`` (model.py:1302-1314)."""
        cfg = self.config
        h = self._conv(x, "decoder.layers.0")
        for stage, ratio in enumerate(cfg.upsampling_ratios):
            h = elu(h)
            h = self._convt(h, f"decoder.layers.{self.dec_up[stage]}", stride=ratio)
            for r, li in enumerate(self.dec_res[stage]):
                h = self._resblock(h, f"decoder.layers.{li}", cfg.dilation_growth_rate ** r)
        h = elu(h)
        return self._conv(h, f"decoder.layers.{self.dec_last}")

    # ---------------- transformer (model.py:1454-2232) ----------------
    def rope_tables(self, batch, length, offset=0):
        """``MimiRotaryEmbedding`` (model.py:1484-1535) for positions
        offset .. offset+T-1 (a streaming chunk starts at the cache length,
        model.py:2179-2186)."""
        cfg = self.config
        inv_freq = 1.0 / (cfg.rope_theta ** (
            torch.arange(0, cfg.head_dim, 2, dtype=torch.int64).float() / cfg.head_dim))
        positions = torch.arange(offset, offset + length).unsqueeze(0).expand(batch, -1)
        inv = inv_freq[None, :, None].float().expand(batch, -1, 1)
        freqs = (inv.float() @ positions[:, None, :].float()).transpose(1, 2)
        emb = torch.cat((freqs, freqs), dim=-1)
        return emb.cos(), emb.sin()

    def attention_mask(self, batch, length):
        """``_attention_mask`` (model.py:1627-1688), sdpa backend, no cache.

        Returns ``None`` (SDPA ``is_causal``) when T < window, else the boolean
        window mask: key k visible from query q iff q - window < k <= q.
        """
        window = self.config.sliding_window
        if length < window:
            return None
        q = torch.arange(length)[:, None]
        k = torch.arange(length)[None, :]
        allowed = (k <= q) & (k > q - window)
        return allowed[None, None].expand(batch, 1, length, length)

    @staticmethod
    def _rotate_half(x):
        a, b = x.chunk(2, dim=-1)
        return torch.cat((-b, a), dim=-1)

    def transformer(self, hidden, prefix):
        """``MimiTransformerModel.forward`` + ``MimiTransformerLayer.forward``
        (model.py:2129-2232, :2028-2061), sdpa backend, no cache."""
        cfg = self.config
        b, t, _ = hidden.shape
        cos, sin = self.rope_tables(b, t)
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
        mask = self.attention_mask(b, t)
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        for i in range(cfg.num_hidden_layers):
            p = f"{prefix}.layers.{i}"
            x = F.layer_norm(hidden, (cfg.hidden_size,), self._w(f"{p}.input_layernorm.weight"),
                             self._w(f"{p}.input_layernorm.bias"), cfg.norm_eps)
            q = F.linear(x, self._w(f"{p}.self_attn.q_proj.weight")).view(b, t, nh, hd).transpose(1, 2)
            k = F.linear(x, self._w(f"{p}.self_attn.k_proj.weight")).view(b, t, nkv, hd).transpose(1, 2)
            v = F.linear(x, self._w(f"{p}.self_attn.v_proj.weight")).view(b, t, nkv, hd).transpose(1, 2)
            q, k = q * cos + self._rotate_half(q) * sin, k * cos + self._rotate_half(k) * sin
            if nh != nkv:
                rep = nh // nkv
                k = k[:, :, None].expand(b, nkv, rep, t, hd).reshape(b, nh, t, hd)
                v = v[:, :, None].expand(b, nkv, rep, t, hd).reshape(b, nh, t, hd)
            o = F.scaled_dot_product_attention(
                q, k, v, attn_mask=mask, dropout_p=0.0, scale=1.0 / math.sqrt(hd),
                is_causal=(t > 1 and mask is None))
            o = o.transpose(1, 2).contiguous()
            o = F.linear(o.reshape(b, t, -1).contiguous(), self._w(f"{p}.self_attn.o_proj.weight"))
            hidden = hidden + self._w(f"{p}.self_attn_layer_scale.scale") * o
            x = F.layer_norm(hidden, (cfg.hidden_size,), self._w(f"{p}.post_attention_layernorm.weight"),
                             self._w(f"{p}.post_attention_layernorm.bias"), cfg.norm_eps)
            m = F.linear(F.gelu(F.linear(x, self._w(f"{p}.mlp.fc1.weight"))), self._w(f"{p}.mlp.fc2.weight"))
            hidden = hidden + self._w(f"{p}.mlp_layer_scale.scale") * m
        return hidden

    # ---------------- streaming (model.py:363-621, :697-797, :2129-2232, :2964-3202) ----------------
    def _conv_stream(self, x, prefix, state, stride=1, dilation=1, pad_mode="constant"):
        """``MimiConv1d.forward`` with a padding cache (model.py:764-797) and
        ``MimiConv1dPaddingCache.update`` (model.py:536-620): the layer sees
        its cached left context followed by the chunk, with no right padding;
        the cache keeps the last ``k_eff - stride`` samples of that input.
        The first chunk's context is zeros, or its first sample repeated for
        replicate padding."""
        w = self._w(f"{prefix}.conv.weight")
        pad = (w.shape[-1] - 1) * dilation + 1 - stride
        ctx = state.conv.get(prefix)
        if ctx is None:
            if pad_mode == "constant":
                ctx = x.new_zeros((x.shape[0], x.shape[1], pad))
            elif pad_mode == "replicate":
                ctx = x[..., :1].expand(x.shape[0], x.shape[1], pad).clone()
            else:
                raise NotImplementedError(f"padding mode {pad_mode!r} is not supported for streaming")
        xx = torch.cat((ctx, x), dim=-1)
        state.conv[prefix] = xx[..., xx.shape[-1] - pad:] if pad > 0 else x.new_empty((x.shape[0], x.shape[1], 0))
        return F.conv1d(xx, w, self.state.get(f"{prefix}.conv.bias"), stride, 0, dilation)

    def _resblock_stream(self, x, prefix, dilation, state):
        h = self._conv_stream(elu(x), f"{prefix}.block.1", state, dilation=dilation)
        h = self._conv_stream(elu(h), f"{prefix}.block.3", state)
        residual = x
        if self.config.use_conv_shortcut:
            residual = self._conv_stream(x, f"{prefix}.shortcut", state)
        return residual + h

    def encoder_stream(self, x, state):
        """``MimiEncoder._forward_eager`` with a padding cache (model.py:1067-1084)."""
        cfg = self.config
        h = self._conv_stream(x, "encoder.layers.0", state)
        for stage, ratio in enumerate(reversed(cfg.upsampling_ratios)):
            for r, li in enumerate(self.enc_res[stage]):
                h = self._resblock_stream(h, f"encoder.layers.{li}", cfg.dilation_growth_rate ** r, state)
            h = elu(h)
            h = self._conv_stream(h, f"encoder.layers.{self.enc_down[stage]}", state, stride=ratio)
        h = elu(h)
        return self._conv_stream(h, f"encoder.layers.{self.enc_last}", state)

    def transformer_cached(self, hidden, prefix, kv):
        """``MimiTransformerModel.forward`` with a ``MimiKVCache``
        (model.py:2129-2232, :363-518): positions continue from the cache
        length; each layer attends to its retained ``window - 1`` rotated
        keys/values plus the chunk; the explicit window mask is skipped in
        exactly the cases ``_attention_mask`` skips it (model.py:1627-1688),
        SDPA then being causal for more than one query (model.py:1846-1866)."""
        cfg = self.config
        b, t, _ = hidden.shape
        window = cfg.sliding_window
        past = kv.length
        cos, sin = self.rope_tables(b, t, offset=past)
        cos, sin = cos.unsqueeze(1), sin.unsqueeze(1)
        key_offset = max(past - window + 1, 0)
        key_length = (window - 1 + t) if past >= window else past + t
        if key_length < window and (t == 1 or key_length == t or past == 0):
            mask = None
        else:
            qp = torch.arange(t)[:, None] + past
            kp = torch.arange(key_length)[None, :] + key_offset
            mask = ((kp <= qp) & (kp > qp - window))[None, None].expand(b, 1, t, key_length)
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        for i in range(cfg.num_hidden_layers):
            p = f"{prefix}.layers.{i}"
            x = F.layer_norm(hidden, (cfg.hidden_size,), self._w(f"{p}.input_layernorm.weight"),
                             self._w(f"{p}.input_layernorm.bias"), cfg.norm_eps)
            q = F.linear(x, self._w(f"{p}.self_attn.q_proj.weight")).view(b, t, nh, hd).transpose(1, 2)
            k = F.linear(x, self._w(f"{p}.self_attn.k_proj.weight")).view(b, t, nkv, hd).transpose(1, 2)
            v = F.linear(x, self._w(f"{p}.self_attn.v_proj.weight")).view(b, t, nkv, hd).transpose(1, 2)
            q, k = q * cos + self._rotate_half(q) * sin, k * cos + self._rotate_half(k) * sin
            if kv.keys[i] is not None:
                k = torch.cat((kv.keys[i], k), dim=-2)
                v = torch.cat((kv.values[i], v), dim=-2)
            keep = window - 1
            kv.keys[i] = k[..., -keep:, :] if keep > 0 else k[..., :0, :]
            kv.values[i] = v[..., -keep:, :] if keep > 0 else v[..., :0, :]
            n = k.shape[-2]
            if nh != nkv:
                rep = nh // nkv
                k = k[:, :, None].expand(b, nkv, rep, n, hd).reshape(b, nh, n, hd)
                v = v[:, :, None].expand(b, nkv, rep, n, hd).reshape(b, nh, n, hd)
            o = F.scaled_dot_product_attention(
                q, k, v, attn_mask=mask, dropout_p=0.0, scale=1.0 / math.sqrt(hd),
                is_causal=(t > 1 and mask is None))
            o = o.transpose(1, 2).contiguous()
            o = F.linear(o.reshape(b, t, -1).contiguous(), self._w(f"{p}.self_attn.o_proj.weight"))
            hidden = hidden + self._w(f"{p}.self_attn_layer_scale.scale") * o
            x = F.layer_norm(hidden, (cfg.hidden_size,), self._w(f"{p}.post_attention_layernorm.weight"),
                             self._w(f"{p}.post_attention_layernorm.bias"), cfg.norm_eps)
            m = F.linear(F.gelu(F.linear(x, self._w(f"{p}.mlp.fc1.weight"))), self._w(f"{p}.mlp.fc2.weight"))
            hidden = hidden + self._w(f"{p}.mlp_layer_scale.scale") * m
        kv.length += t
        return hidden

    @torch.inference_mode()
    def encode_stream(self, chunk, num_quantizers, state, trace=None):
        """One ``encode(..., use_streaming=True)`` call (model.py:3070-3137,
        :2964-3005): SEANet encoder and downsample on padding caches, encoder
        transformer on its KV cache, then the (stateless) split RVQ."""
        emb = self.encoder_stream(chunk, state)
        h = self.transformer_cached(emb.transpose(1, 2), "encoder_transformer", state.encoder_kv)
        emb = h.transpose(1, 2)
        if self._bottleneck_ratio() is not None:
            emb = self._conv_stream(emb, "downsample", state, stride=2, pad_mode="replicate")
        return self.quantizer_encode(emb, num_quantizers, trace)

    @torch.inference_mode()
    def decode_cached(self, codes, kv):
        """``decode(codes, decoder_past_key_values=kv)`` (model.py:3139-3202):
        only the decoder transformer carries state; RVQ decode, upsample and
        the SEANet decoder run on the chunk alone."""
        emb = self.quantizer_decode(codes)
        if self._bottleneck_ratio() is not None:
            emb = self._convt(emb, "upsample", stride=2, groups=self.config.upsample_groups)
        h = self.transformer_cached(emb.transpose(1, 2), "decoder_transformer", kv)
        return self.decoder(h.transpose(1, 2))

    def new_stream(self):
        return StreamState(encoder_kv=KVState(self.config.num_hidden_layers))

    def new_kv(self):
        return KVState(self.config.num_hidden_layers)

    # ---------------- quantizer (model.py:2238-2696) ----------------
    def embed(self, codebook_prefix):
        """``MimiEuclideanCodebook.embed`` (model.py:2263-2275)."""
        e = self._embeds.get(codebook_prefix)
        if e is None:
            usage = self._w(f"{codebook_prefix}.cluster_usage").clamp(min=1e-5)
            e = self._w(f"{codebook_prefix}.embed_sum") / usage[:, None]
            self._embeds[codebook_prefix] = e
        return e

    @staticmethod
    def nearest(rows, embed):
        """``MimiEuclideanCodebook.quantize`` (model.py:2277-2291):
        ``cdist(...).argmin(-1)`` — lowest index wins ties."""
        d = torch.cdist(rows[None].float(), embed[None].float(), p=2)[0]
        return d.argmin(dim=-1)

    def _rvq_encode(self, emb, prefix, count, trace):
        """``MimiResidualVectorQuantizer.encode`` (model.py:2408-2428)."""
        proj = self.state.get(f"{prefix}.input_proj.weight")
        x = F.conv1d(emb, proj) if proj is not None else emb
        residual = x
        out = []
        for j in range(count):
            e = self.embed(f"{prefix}.layers.{j}.codebook")
            rows = residual.permute(0, 2, 1)
            flat = rows.reshape(-1, rows.shape[-1])
            if trace is not None:
                trace.rvq_inputs.append((f"{prefix}.layers.{j}", flat.clone()))
            idx = self.nearest(flat, e).view(rows.shape[:-1])
            residual = residual - F.embedding(idx, e).permute(0, 2, 1)
            out.append(idx)
        return torch.stack(out)

    def quantizer_encode(self, emb, count, trace=None):
        """``MimiSplitResidualVectorQuantizer._encode_eager`` + range checks
        (model.py:2485-2501, :2570-2593); returns ``[B, nq, T]``."""
        cfg = self.config
        if count > cfg.num_quantizers:
            raise ValueError(f"num_quantizers must be <= {cfg.num_quantizers}, got {count}")
        if count < cfg.num_semantic_quantizers:
            raise ValueError(f"num_quantizers must be >= {cfg.num_semantic_quantizers}, got {count}")
        sem = "quantizer.semantic_residual_vector_quantizer"
        ac = "quantizer.acoustic_residual_vector_quantizer"
        codes = self._rvq_encode(emb, sem, cfg.num_semantic_quantizers, trace)
        if count > cfg.num_semantic_quantizers:
            codes = torch.cat((codes, self._rvq_encode(emb, ac, count - cfg.num_semantic_quantizers, trace)), 0)
        return codes.transpose(0, 1)

    def _rvq_decode(self, codes, prefix):
        """``MimiResidualVectorQuantizer.decode`` (model.py:2430-2444): float32
        zero plus codebooks left to right, then ``output_proj``."""
        q = codes.new_zeros((), dtype=torch.float32)
        for j, idx in enumerate(codes.transpose(0, 1)):
            q = q + F.embedding(idx, self.embed(f"{prefix}.layers.{j}.codebook")).permute(0, 2, 1)
        proj = self.state.get(f"{prefix}.output_proj.weight")
        return F.conv1d(q, proj) if proj is not None else q

    def quantizer_decode(self, codes):
        """``MimiSplitResidualVectorQuantizer._decode_eager`` (model.py:2611-2627)."""
        ns = self.config.num_semantic_quantizers
        out = self._rvq_decode(codes[:, :ns], "quantizer.semantic_residual_vector_quantizer")
        if codes.shape[1] > ns:
            out = out + self._rvq_decode(codes[:, ns:], "quantizer.acoustic_residual_vector_quantizer")
        return out

    # ---------------- composition (model.py:2964-3268) ----------------
    def _bottleneck_ratio(self):
        cfg = self.config
        if cfg.frame_rate == cfg.encodec_frame_rate:
            return None
        return int(cfg.encodec_frame_rate / cfg.frame_rate)

    def encode(self, audio, num_quantizers=None, trace=None):
        """``MimiModel._encode_frame`` (model.py:2964-3005)."""
        cfg = self.config
        count = cfg.num_quantizers if num_quantizers is None else num_quantizers
        if count > cfg.num_quantizers:
            raise ValueError(f"num_quantizers must be <= {cfg.num_quantizers}, got {count}")
        if audio.ndim != 3:
            raise ValueError("input_values must have shape [batch, channels, samples]")
        if not 1 <= audio.shape[1] <= 2:
            raise ValueError("input audio must have one or two channels")
        emb = self.encoder(audio)
        if trace is not None:
            trace.encoder_out = emb
        h = self.transformer(emb.transpose(1, 2), "encoder_transformer")
        if trace is not None:
            trace.transformer_out = h
        emb = h.transpose(1, 2)
        if self._bottleneck_ratio() is not None:
            emb = self._conv(emb, "downsample", stride=2, pad_mode="replicate")
        if trace is not None:
            trace.downsampled = emb
        return self.quantizer_encode(emb, count, trace)

    def decode(self, codes, padding_mask=None, trace=None):
        """``MimiModel._decode_frame`` + crop (model.py:3139-3199)."""
        emb = self.quantizer_decode(codes)
        if trace is not None:
            trace.quantized = emb
        if self._bottleneck_ratio() is not None:
            emb = self._convt(emb, "upsample", stride=2, groups=self.config.upsample_groups)
        h = self.transformer(emb.transpose(1, 2), "decoder_transformer")
        if trace is not None:
            trace.decoder_in = h
        audio = self.decoder(h.transpose(1, 2))
        if padding_mask is not None and padding_mask.shape[-1] < audio.shape[-1]:
            audio = audio[..., : padding_mask.shape[-1]]
        return audio

    @torch.inference_mode()
    def forward(self, audio, padding_mask=None, num_quantizers=None, trace=None):
        """``MimiModel._forward_eager`` (model.py:3204-3268): the mask is only
        used to crop the decoded waveform (encode ignores it, :3123-3134)."""
        if padding_mask is None:
            padding_mask = torch.ones_like(audio, dtype=torch.bool)
        codes = self.encode(audio, num_quantizers, trace)
        return codes, self.decode(codes, padding_mask, trace)

    def encoded_length(self, lengths):
        """``MimiModel.get_encoded_length`` (model.py:3007-3024), closed form."""
        cfg = self.config
        out = []
        for n in lengths:
            n = int(n)
            n = conv_output_length(n, cfg.kernel_size, 1)
            for ratio in reversed(cfg.upsampling_ratios):
                for _ in range(cfg.num_residual_layers):
                    n = conv_output_length(n, cfg.residual_kernel_size, 1)
                    n = conv_output_length(n, 1, 1)
                n = conv_output_length(n, 2 * ratio, ratio)
            n = conv_output_length(n, cfg.last_kernel_size, 1)
            r = self._bottleneck_ratio()
            if r is not None:
                n = conv_output_length(n, 2 * r, 2)
            out.append(n)
        return out


def rvq_margins(oracle: MimiOracle, trace: Trace):
    """Per codebook and query row, (best, second-best) squared distances in
    float64 and the gap between them relative to |x|^2 + |e|^2 — the scale of
    FP32 rounding in the reference's mm-form cdist.  Diagnostics only."""
    out = []
    for prefix, rows in trace.rvq_inputs:
        e = oracle.embed(f"{prefix}.codebook").double()
        x = rows.double()
        d2 = (x * x).sum(-1, keepdim=True) + (e * e).sum(-1)[None] - 2.0 * x @ e.T
        top = torch.topk(d2, 2, dim=-1, largest=False)
        scale = (x * x).sum(-1) + (e * e).sum(-1)[top.indices[:, 0]]
        gap = (top.values[:, 1] - top.values[:, 0]) / scale
        out.append((prefix, top.indices, gap))
    return out
