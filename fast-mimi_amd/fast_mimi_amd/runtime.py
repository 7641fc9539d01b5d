"""Device runtime: packed weights and the layer sequence of encode / decode.

Every contraction and every nonlinearity runs in ``libfast_mimi_amd.so``;
PyTorch only owns device memory (weights, activations, workspaces) and the
stream.  Activations are channels-last ``[batch, positions, channels]``
throughout, so the reference's NCL ``transpose(1, 2)`` hand-offs between the
SEANet stacks and the transformers (``model.py:2964-3005``, ``:3139-3170``)
disappear.

Fusion plan (one kernel per line):
  SEANet conv           -> implicit GEMM + bias (+ ELU when an ELU follows)
  residual block conv1  -> ELU-on-load + k3 conv + bias + ELU
  residual block conv2  -> 1x1 conv + bias + residual add (+ ELU when one follows)
  ConvTranspose1d       -> stride-phase GEMM + bias
  LayerNorm             -> one wave per row
  q/k/v projections     -> one GEMM against the packed [hidden, 3*hidden] weight
  attention             -> RoPE on load + causal window-250 online softmax
  o_proj / fc2          -> GEMM + LayerScale residual (in place)
  fc1                   -> GEMM + exact-erf GELU
  RVQ in projections    -> one GEMM for both branches
  RVQ codebook step     -> distance GEMM + argmin + residual subtract
  RVQ decode            -> ordered gather-sum, then one GEMM for both out projections
"""

from __future__ import annotations

import threading

import torch

from . import _native as nat
from . import ops
from .config import MimiConfig
from .flops import layer_table
from .weights import decoder_layer_indices, encoder_layer_indices

_WORKSPACE_BYTES = 64 << 20


# Up to this many rows the transformer projections run as row-block kernels with
# LayerNorm / RoPE fused; above it, tiled GEMMs amortise the weight reads better.
_ROW_LINEAR_MAX_ROWS = 1024
# Up to this many rows the 16-row kernels on fragment-packed weights are used.
_ROW16_MAX_ROWS = 512
# Few-row long-K convolutions (fm_conv1d_rows) up to this many multiply-adds
# (rows x out x K); beyond it the tiled GEMM engine has enough tiles.  Measured
# at C2 shapes (warm, us, split GEMM -> row blocks): encoder last conv 21.1 ->
# 12.6, downsample 12.2 -> 8.4, decoder first conv 27.9 -> 25.1, 512-channel
# residual block's k3 conv at 2000 rows 27.2 -> 21.8; at 1.6e9 MACs and above
# the row blocks lose (the 512-channel k3 conv at 4000 rows 34.2 -> 40.9).
_ROWCONV_MAX_MACS = 1_000_000_000


class _Conv:
    """Causal Conv1d packed for the implicit GEMM as W^T[c_out, (tap, c_in)]."""

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, stride: int = 1,
                 pad_mode: str = "constant"):
        c_out, c_in, k = weight.shape
        self.c_in, self.c_out, self.k, self.stride = c_in, c_out, k, stride
        self.replicate = 1 if pad_mode == "replicate" else 0
        self.w = weight.permute(0, 2, 1).reshape(c_out, k * c_in).contiguous()
        self.b = None if bias is None else bias.contiguous()
        self.flags = 0  # nat.WEIGHTS_X6 once the runtime appends the bf16 planes
        self.wr = None  # fragment-packed W^T for fm_conv1d_rows, where that kernel applies


class _ConvT:
    """Causal ConvTranspose1d packed as W^T[(phase, c_out), (tap, c_in)].

    Output row q*s + r reads inputs q - taps + 1 .. q; window slot jj holds input
    q - (taps - 1 - jj), which meets kernel tap r + (taps - 1 - jj) * s.
    """

    def __init__(self, weight: torch.Tensor, bias: torch.Tensor | None, stride: int):
        c_in, c_out, k = weight.shape
        if k % stride:
            raise ValueError("transposed-conv kernel must be a multiple of its stride")
        taps = k // stride
        self.c_in, self.c_out, self.k, self.stride = c_in, c_out, k, stride
        w = weight.reshape(c_in, c_out, taps, stride).flip(2)  # [ci, co, jj, r]
        self.w = w.permute(3, 1, 2, 0).reshape(stride * c_out, taps * c_in).contiguous()
        self.b = None if bias is None else bias.contiguous()
        self.flags = 0


class _Layer:
    def __init__(self, state, prefix, cfg: MimiConfig):
        g = lambda n: state[f"{prefix}.{n}"]  # noqa: E731
        self.ln1 = (g("input_layernorm.weight").contiguous(), g("input_layernorm.bias").contiguous())
        self.ln2 = (g("post_attention_layernorm.weight").contiguous(),
                    g("post_attention_layernorm.bias").contiguous())
        # Linear weights are [out, in] = W^T already.
        self.wqkv = torch.cat([g("self_attn.q_proj.weight"), g("self_attn.k_proj.weight"),
                               g("self_attn.v_proj.weight")], 0).contiguous()
        self.wo = g("self_attn.o_proj.weight").contiguous()
        self.w1 = g("mlp.fc1.weight").contiguous()
        self.w2 = g("mlp.fc2.weight").contiguous()
        self.ls1 = g("self_attn_layer_scale.scale").contiguous()
        self.ls2 = g("mlp_layer_scale.scale").contiguous()


_PROJECTIONS = ("qkv", "o", "fc1", "fc2")


def x6_plan(config: MimiConfig) -> dict[str, bool]:
    """Which contractions carry bf16x6 weight planes, by ``flops.layer_table``
    name: every SEANet conv / transposed conv and every transformer projection
    whose reduction length K (the packed weight's row length) is a multiple of
    16, the k-tile of the planes.  The RVQ projections keep FP32 weights only.
    Independent of batch and length; the runtime checks itself against it."""
    plan = {}
    for name, kind, _, _, k, _ in layer_table(config, 1, 2 * config.sampling_rate, 1):
        if kind in ("conv", "convt") or (kind == "gemm" and name.rsplit(".", 1)[-1] in _PROJECTIONS):
            plan[name] = k % 16 == 0
    return plan


def rope_tables(config: MimiConfig, length: int) -> tuple[torch.Tensor, torch.Tensor]:
    """cos/sin ``[T, head_dim]`` exactly as ``MimiRotaryEmbedding`` builds them
    (``model.py:1499-1535``): float32 inverse frequencies, one rounded product
    per (position, frequency), duplicated halves, CPU ``cos``/``sin``."""
    d = config.head_dim
    inv_freq = 1.0 / (config.rope_theta ** (torch.arange(0, d, 2, dtype=torch.int64).float() / d))
    freqs = torch.arange(length).float()[:, None] * inv_freq[None, :]
    emb = torch.cat((freqs, freqs), dim=-1)
    return emb.cos().contiguous(), emb.sin().contiguous()


class MimiRuntime:
    """Executes Mimi encode / decode on one GPU through the HIP library."""

    def __init__(self, config: MimiConfig, state: dict[str, torch.Tensor], device: torch.device):
        if config.use_conv_shortcut:
            raise NotImplementedError("learned residual shortcuts are not part of this runtime")
        if config.num_residual_layers != 1:
            raise NotImplementedError("only one residual block per SEANet stage (dilation 1) is supported")
        if config.vector_quantization_hidden_dimension == config.hidden_size:
            raise NotImplementedError("RVQ without input/output projections is not supported")
        nat.library()
        self.config = config
        self.device = device
        self.lock = threading.Lock()
        st = {k: v.to(device=device, dtype=torch.float32) for k, v in state.items()}
        cfg = config

        def conv(prefix, stride=1, pad_mode="constant"):
            return _Conv(st[f"{prefix}.conv.weight"], st.get(f"{prefix}.conv.bias"), stride, pad_mode)

        def res(prefix):
            return (conv(f"{prefix}.block.1"), conv(f"{prefix}.block.3"))

        enc = encoder_layer_indices(cfg)
        ratios = list(reversed(cfg.upsampling_ratios))
        self.enc_first = conv("encoder.layers.0")
        self.enc_stages = [(res(f"encoder.layers.{enc['res'][i][0]}"),
                            conv(f"encoder.layers.{enc['down'][i]}", stride=r))
                           for i, r in enumerate(ratios)]
        self.enc_last = conv(f"encoder.layers.{enc['last'][0]}")
        dec = decoder_layer_indices(cfg)
        self.dec_first = conv("decoder.layers.0")
        self.dec_stages = [(_ConvT(st[f"decoder.layers.{dec['up'][i]}.conv.weight"],
                                   st.get(f"decoder.layers.{dec['up'][i]}.conv.bias"), r),
                            res(f"decoder.layers.{dec['res'][i][0]}"))
                           for i, r in enumerate(cfg.upsampling_ratios)]
        self.dec_last = conv(f"decoder.layers.{dec['last'][0]}")
        self.enc_tf = [_Layer(st, f"encoder_transformer.layers.{i}", cfg) for i in range(cfg.num_hidden_layers)]
        self.dec_tf = [_Layer(st, f"decoder_transformer.layers.{i}", cfg) for i in range(cfg.num_hidden_layers)]
        self.bottleneck = cfg.frame_rate != cfg.encodec_frame_rate
        if self.bottleneck:
            self.down = conv("downsample", stride=2, pad_mode="replicate")
            self.up_w = st["upsample.conv.weight"].contiguous()
            self.up_k = self.up_w.shape[-1]
            if cfg.upsample_groups != cfg.hidden_size:
                raise NotImplementedError("only a depthwise bottleneck upsample is supported")

        # Quantizer: both in-projections as one GEMM, both out-projections as one.
        sem = "quantizer.semantic_residual_vector_quantizer"
        ac = "quantizer.acoustic_residual_vector_quantizer"
        self.vq = cfg.vector_quantization_hidden_dimension
        self.w_in = torch.cat([st[f"{sem}.input_proj.weight"][:, :, 0],
                               st[f"{ac}.input_proj.weight"][:, :, 0]], 0).contiguous()
        self.w_out = torch.cat([st[f"{sem}.output_proj.weight"][:, :, 0],
                                st[f"{ac}.output_proj.weight"][:, :, 0]], 1).contiguous()
        n_sem = cfg.num_semantic_quantizers
        prefixes = [f"{sem}.layers.{j}.codebook" for j in range(n_sem)]
        prefixes += [f"{ac}.layers.{j}.codebook" for j in range(cfg.num_quantizers - n_sem)]
        e, d = cfg.codebook_size, cfg.codebook_dim
        self.embeds = torch.empty((len(prefixes), e, d), device=device)
        self.embeds_t = torch.empty((len(prefixes), d, e), device=device)
        self.norms = torch.empty((len(prefixes), e), device=device)
        for j, p in enumerate(prefixes):
            ops.call("fm_rvq_prepare_codebook", st[f"{p}.embed_sum"].contiguous(),
                     st[f"{p}.cluster_usage"].contiguous(), e, d, 1e-5,
                     self.embeds[j], self.embeds_t[j],
                     self.norms[j])
        # Fragment-packed copies of the projection weights for the few-row kernels,
        # keyed by the row-major weight's device address.
        self._packed: dict[int, torch.Tensor] = {}
        lib = nat.library()
        for w in [m for lay in self.enc_tf + self.dec_tf for m in (lay.wqkv, lay.wo, lay.w1, lay.w2)] + \
                [self.w_in, self.w_out]:
            n, k = w.shape
            if lib.fm_row_linear_supported(k, n):
                pw = torch.empty_like(w)
                ops.call("fm_pack_row_weights", w, n, k, pw)
                self._packed[w.data_ptr()] = pw
        # Convolution and large-row projection weights carry their bf16x6
        # planes: W^T followed by [3][N][K] bf16 in one buffer.
        self._x6: dict[int, torch.Tensor] = {}
        for layer in self._conv_layers():
            w = self._with_planes(layer.w)
            if w is not layer.w:
                layer.w, layer.flags = w, nat.WEIGHTS_X6
        for w in [m for lay in self.enc_tf + self.dec_tf for m in (lay.wqkv, lay.wo, lay.w1, lay.w2)]:
            self._x6[w.data_ptr()] = self._with_planes(w)
        # Which layers took planes, checked against the declared plan (a layer
        # without planes would silently run its FP32 kernels instead).
        self.x6_layers = {name: bool(layer.flags & nat.WEIGHTS_X6) for name, layer in self._named_conv_layers()}
        for tag, layers in (("enc.tf", self.enc_tf), ("dec.tf", self.dec_tf)):
            for i, lay in enumerate(layers):
                for short, w in zip(_PROJECTIONS, (lay.wqkv, lay.wo, lay.w1, lay.w2)):
                    self.x6_layers[f"{tag}{i}.{short}"] = self._x6[w.data_ptr()] is not w
        if self.x6_layers != x6_plan(cfg):
            raise RuntimeError("bf16x6 weight planes do not follow x6_plan: "
                               f"{sorted(set(self.x6_layers.items()) ^ set(x6_plan(cfg).items()))}")
        # Few-row long-K convolutions (fm_conv1d_rows, see _ROWCONV_MAX_MACS):
        # on the bf16x6 planes where the layer has them, else on
        # fragment-packed FP32 weights.
        for layer in self._conv_layers():
            if layer.flags & nat.WEIGHTS_X6 and lib.fm_conv1d_rows_supported(
                    layer.c_in, layer.c_out, layer.k, nat.WEIGHTS_X6):
                layer.wr = layer.w
            elif lib.fm_conv1d_rows_supported(layer.c_in, layer.c_out, layer.k, 0):
                layer.wr = torch.empty_like(layer.w)
                ops.call("fm_pack_row_weights", layer.w, layer.c_out, layer.k * layer.c_in, layer.wr)
        self.workspace = torch.empty(_WORKSPACE_BYTES // 4, device=device)
        self._rope: dict[int, tuple[torch.Tensor, torch.Tensor]] = {}
        # Optional per-op timing: a list of (tag, start_event, end_event).
        self.profile: list | None = None
        self._tag = ""
        torch.cuda.synchronize(device)

    def _named_conv_layers(self):
        """(``flops.layer_table`` name, layer) of every SEANet / bottleneck conv."""
        cfg = self.config
        out = [("enc.first", self.enc_first)]
        ch = cfg.num_filters
        for r, ((c1, c2), down) in zip(reversed(cfg.upsampling_ratios), self.enc_stages):
            out += [(f"enc.res{ch}.c1", c1), (f"enc.res{ch}.c2", c2), (f"enc.down{r}", down)]
            ch *= 2
        out.append(("enc.last", self.enc_last))
        if self.bottleneck:
            out.append(("down", self.down))
        out.append(("dec.first", self.dec_first))
        for r, (convt, (c1, c2)) in zip(cfg.upsampling_ratios, self.dec_stages):
            out += [(f"dec.up{r}", convt), (f"dec.res{convt.c_out}.c1", c1), (f"dec.res{convt.c_out}.c2", c2)]
        out.append(("dec.last", self.dec_last))
        return out

    def _conv_layers(self):
        return [layer for _, layer in self._named_conv_layers()]

    def _with_planes(self, w: torch.Tensor) -> torch.Tensor:
        """``w`` [N, K] (FP32 W^T) as the first N*K floats of a buffer that
        continues with its three bf16 planes (``fm_split_weights``); ``w``
        itself when K is not a multiple of 16."""
        rows, cols = w.shape
        if cols % 16:
            return w
        n = w.numel()
        buf = torch.empty(n + 3 * n // 2, device=self.device)
        buf[:n].copy_(w.reshape(-1))
        ops.call("fm_split_weights", buf[:n], rows, cols, buf[n:])
        return buf[:n].view(w.shape)

    # ------------------------------------------------------------------ ops
    def _call(self, name: str, *args) -> None:
        """Run C-ABI entry point ``name`` through its ``torch.ops.fast_mimi_amd``
        operator on the current stream (tensors in place of device pointers)."""
        if self.profile is None:
            ops.call(name, *args)
            return
        start = torch.cuda.Event(enable_timing=True)
        stop = torch.cuda.Event(enable_timing=True)
        start.record()
        ops.call(name, *args)
        stop.record()
        self.profile.append((f"{self._tag}:{name}", start, stop))

    def profile_report(self) -> list[tuple[str, float]]:
        """(tag, milliseconds) per recorded op; clears the record."""
        torch.cuda.synchronize(self.device)
        out = [(tag, a.elapsed_time(b)) for tag, a, b in (self.profile or [])]
        self.profile = [] if self.profile is not None else None
        return out

    def _conv(self, x, B, L, layer: _Conv, flags=0, residual=None, y_len=None):
        rows = -(-L // layer.stride)
        y_len = rows if y_len is None else y_len
        y = torch.empty((B, y_len, layer.c_out), device=self.device)
        if (layer.wr is not None and y_len == rows
                and B * rows * layer.c_out * layer.k * layer.c_in <= _ROWCONV_MAX_MACS
                and not flags & ~(nat.ELU_IN | nat.EPI_ELU | nat.EPI_RES_ADD)):
            self._call("fm_conv1d_rows", x, B, L, layer.c_in, layer.wr, layer.b, layer.c_out,
                       layer.c_out, layer.k, layer.stride, layer.replicate,
                       flags | (layer.flags if layer.wr is layer.w else 0), residual, y)
            return y, rows
        self._call("fm_conv1d", x, B, L, layer.c_in, layer.w, layer.b,
                 layer.c_out, layer.k, layer.stride, layer.replicate, flags | layer.flags, residual,
                 y, y_len, self.workspace, _WORKSPACE_BYTES)
        return y, rows

    def _convt(self, x, B, L, layer: _ConvT):
        y = torch.empty((B, L * layer.stride, layer.c_out), device=self.device)
        self._call("fm_conv_transpose1d", x, B, L, layer.c_in, layer.w,
                 layer.b, layer.c_out, layer.k, layer.stride, layer.flags, None, y,
                 self.workspace, _WORKSPACE_BYTES)
        return y, L * layer.stride

    def _linear(self, x, rows, w, flags=0, residual=None, scale=None, out=None):
        n, k = w.shape
        y = torch.empty((rows, n), device=self.device) if out is None else out
        wx = self._x6.get(w.data_ptr())
        if wx is not None:
            w, flags = wx, flags | nat.WEIGHTS_X6
        self._call("fm_linear", x, rows, k, w, n, flags, residual,
                 scale, y, self.workspace, _WORKSPACE_BYTES)
        return y

    def _linear_rope(self, x, rows, w, cos, sin, rope_cols, per_seq):
        """q/k/v projection with RoPE in the bf16x6 GEMM's epilogue (the
        attention then reads rotated q / k)."""
        n, k = w.shape
        y = torch.empty((rows, n), device=self.device)
        self._call("fm_linear_rope", x, rows, k, self._x6[w.data_ptr()], n, nat.WEIGHTS_X6, cos, sin,
                   rope_cols, per_seq, y, self.workspace, _WORKSPACE_BYTES)
        return y

    def _proj(self, x, rows, w, flags=0, residual=None, scale=None, out=None):
        """Plain projection: row-block kernel for few rows, tiled GEMM otherwise."""
        n, k = w.shape
        if rows <= _ROW_LINEAR_MAX_ROWS and nat.library().fm_row_linear_supported(k, n):
            return self._row_linear(x, rows, w, flags, residual, scale, out)
        return self._linear(x, rows, w, flags, residual, scale, out)

    def _row_linear(self, x, rows, w, flags=0, residual=None, scale=None, out=None, ln=None,
                    rope=None):
        """Transformer projection with LayerNorm prologue / RoPE epilogue fused."""
        n, k = w.shape
        y = torch.empty((rows, n), device=self.device) if out is None else out
        g, b = (ln[0], ln[1]) if ln is not None else (None, None)
        cos, sin, rope_cols, per_seq = rope if rope is not None else (None, None, 0, 1)
        few = rows <= _ROW16_MAX_ROWS
        # bf16x6 where it measured faster at 250 rows: the wide 512-deep
        # projections (qkv 7.5 vs 9.4 us, fc1 7.7 vs 9.6 us); the output
        # projection (3.5 vs 3.4 us) and the streamed fc2 (8.1 vs 8.1 us)
        # keep the FP32 fragment-packed kernel.
        wx = self._x6.get(w.data_ptr()) if few and k == 512 and n >= 1024 else None
        packed = self._packed.get(w.data_ptr()) if few else None
        if wx is not None:  # 16-row blocks on the bf16 matrix cores (bf16x6)
            name, wp, flags = "fm_row_linear", wx, flags | nat.WEIGHTS_X6
        elif packed is not None:
            name, wp = "fm_row_linear_packed", packed
        else:
            name, wp = "fm_row_linear", w
        self._call(name, x, rows, k, g, b, self.config.norm_eps,
                   wp, n, flags, residual, scale, cos, sin,
                   rope_cols, per_seq, y)
        return y

    def _fuse_last(self, block) -> bool:
        """The decoder's last residual block and waveform conv run as one
        kernel pair when they have the SEANet shapes (64 channels, k = 3)."""
        c1, c2 = block
        last = self.dec_last
        return (c1.k == 3 and c2.c_out == 64 and last.c_in == 64 and last.c_out == 1
                and last.k == 3 and last.stride == 1 and not last.replicate)

    def _resblock(self, x, B, L, block, elu_after: bool, tag: str = "res", act_exp: bool = False):
        """act_exp: the bf16x6 block evaluates its ELUs as e^x - 1 (absolute
        error of a few 1e-8; decoder only: the encoder's codes need exact
        activations)."""
        c1, c2 = block
        # The fused kernel (hidden tile kept on chip) covers the SEANet widths;
        # other shapes run as two GEMM-engine convs.
        fused = c1.k == 3 and nat.library().fm_resblock_supported(c2.c_out)
        if fused:
            self._tag = tag
            y = torch.empty_like(x)
            flags = (1 if elu_after else 0) | (c1.flags & c2.flags & nat.WEIGHTS_X6)
            if act_exp and flags & nat.WEIGHTS_X6:
                flags |= nat.ACT_EXP
            self._call("fm_resblock", x, B, L, c2.c_out, c1.w, c1.b, c2.w, c2.b, flags, y)
            return y
        self._tag = f"{tag}.c1"
        h, _ = self._conv(x, B, L, c1, nat.ELU_IN | nat.EPI_ELU)
        flags = nat.EPI_RES_ADD | (nat.EPI_ELU if elu_after else 0)
        self._tag = f"{tag}.c2"
        y, _ = self._conv(h, B, L, c2, flags, residual=x)
        return y

    def _rope_tables(self, length):
        tabs = self._rope.get(length)
        if tabs is None:
            if torch.cuda.is_current_stream_capturing():
                raise RuntimeError("RoPE tables must be prepared before graph capture")
            c, s = rope_tables(self.config, length)
            tabs = (c.to(self.device), s.to(self.device))
            self._rope[length] = tabs
        return tabs

    def prepare(self, length: int) -> None:
        """Upload the RoPE tables a sequence of ``length`` frames needs."""
        self._rope_tables(length)

    def transformer(self, h, B, T, layers, tag: str = "tf"):
        cfg = self.config
        M = B * T
        C = cfg.hidden_size
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        cos, sin = self._rope_tables(T)
        h = h.reshape(M, C)
        xln = torch.empty((M, C), device=self.device)
        att = torch.empty((M, nh * hd), device=self.device)
        lib = nat.library()
        fused = (M <= _ROW_LINEAR_MAX_ROWS and hd == 64 and lib.fm_row_linear_supported(C, layers[0].wqkv.shape[0])
                 and lib.fm_row_linear_supported(C, layers[0].w1.shape[0])
                 and lib.fm_row_linear_supported(nh * hd, C))
        rope_cols = (nh + nkv) * hd
        for li, lay in enumerate(layers):
            # Above the row-block sizes RoPE rides in the tiled qkv GEMM's
            # epilogue when its weight carries bf16x6 planes (4 us per layer
            # less than rotating in the attention kernels at 2500-4000 rows).
            rope_gemm = (not fused and hd == 64 and rope_cols % 64 == 0
                         and self._x6.get(lay.wqkv.data_ptr(), lay.wqkv) is not lay.wqkv)
            if fused:
                self._tag = f"{tag}{li}.qkv"
                qkv = self._row_linear(h, M, lay.wqkv, ln=lay.ln1, rope=(cos, sin, rope_cols, T))
            else:
                self._tag = f"{tag}{li}.ln1"
                self._call("fm_layer_norm", h, lay.ln1[0],
                           lay.ln1[1], M, C, cfg.norm_eps, xln)
                self._tag = f"{tag}{li}.qkv"
                if rope_gemm:
                    qkv = self._linear_rope(xln, M, lay.wqkv, cos, sin, rope_cols, T)
                else:
                    qkv = self._linear(xln, M, lay.wqkv)
            ld = qkv.shape[1]
            self._tag = f"{tag}{li}.attn"
            tabs = (None, None) if fused or rope_gemm else (cos, sin)
            self._call("fm_window_attention", qkv, ld, 0, nh * hd, (nh + nkv) * hd,
                       tabs[0], tabs[1], B, T, nh, nkv, hd, cfg.sliding_window,
                       1.0 / (hd ** 0.5), att, nh * hd)
            self._tag = f"{tag}{li}.o"
            if fused:
                self._row_linear(att, M, lay.wo, nat.EPI_RES_SCALE, residual=h, scale=lay.ls1, out=h)
                self._tag = f"{tag}{li}.fc1"
                ff = self._row_linear(h, M, lay.w1, nat.EPI_GELU, ln=lay.ln2)
            else:
                self._linear(att, M, lay.wo, nat.EPI_RES_SCALE, residual=h, scale=lay.ls1, out=h)
                self._tag = f"{tag}{li}.ln2"
                self._call("fm_layer_norm", h, lay.ln2[0],
                           lay.ln2[1], M, C, cfg.norm_eps, xln)
                self._tag = f"{tag}{li}.fc1"
                ff = self._linear(xln, M, lay.w1, nat.EPI_GELU)
            self._tag = f"{tag}{li}.fc2"
            self._proj(ff, M, lay.w2, nat.EPI_RES_SCALE, residual=h, scale=lay.ls2, out=h)
        return h.reshape(B, T, C)

    # ------------------------------------------------------------- stages
    def encode(self, audio: torch.Tensor, num_quantizers: int, padding_cache=None,
               kv_cache=None) -> torch.Tensor:
        """``[B, C, S]`` float32 audio -> ``[B, nq, T]`` int64 codes.

        With ``padding_cache`` the convolutions run on cached left context with
        no right padding (streaming); with ``kv_cache`` the transformer
        continues from cached keys/values (``model.py:2964-3005``)."""
        h, B, L = self.embeddings(audio, padding_cache, kv_cache)
        return self.quantize(h, B, L, num_quantizers)

    def embeddings(self, audio: torch.Tensor, padding_cache=None, kv_cache=None):
        """Encoder output entering the quantizer: ``(h [B, T12.5, C], B, T12.5)``."""
        B, C, S = audio.shape
        x = audio if C == 1 else audio.transpose(1, 2).contiguous()
        if padding_cache is None:
            h, L = self._encoder_seanet(x, B, S)
        else:
            h, L = self._encoder_seanet_stream(x.view(B, S, C), B, padding_cache)
        if kv_cache is None:
            h = self.transformer(h, B, L, self.enc_tf, "enc.tf")
        else:
            h = self.transformer_cached(h, B, L, self.enc_tf, kv_cache)
        if self.bottleneck:
            self._tag = "down"
            if padding_cache is None:
                h, L = self._conv(h, B, L, self.down)
            else:
                h, L = self._stream_conv(h, self.down, padding_cache, len(padding_cache.padding_cache) - 1)
        return h, B, L

    def quantizer_inputs(self, h, B, T) -> torch.Tensor:
        """Both branches' projected RVQ inputs ``[B*T, 2*dim]`` (semantic | acoustic)."""
        self._tag = "rvq.in"
        return self._proj(h.reshape(B * T, self.config.hidden_size), B * T, self.w_in)

    def _encoder_seanet(self, x, B, S):
        n = len(self.enc_stages)
        first, (c1, c2) = self.enc_first, self.enc_stages[0][0]
        if (first.c_in == 1 and first.k == 7 and first.stride == 1 and first.c_out == 64
                and not first.replicate and c1.k == 3 and c2.c_out == 64 and first.b is not None):
            # The first conv is formed inside the first residual block.
            self._tag = "enc.first+res64"
            h = torch.empty((B, S, 64), device=self.device)
            self._call("fm_conv_resblock64", x, B, S, first.w,
                       first.b, c1.w, c1.b, c2.w,
                       c2.b, 1 | (c1.flags & c2.flags & nat.WEIGHTS_X6), h)
            L, start = S, 1
        else:
            self._tag = "enc.first"
            h, L = self._conv(x, B, S, self.enc_first)
            start = 0
        for i, (block, down) in enumerate(self.enc_stages):
            if i >= start:
                h = self._resblock(h, B, L, block, elu_after=True, tag=f"enc.res{down.c_in}")
            self._tag = f"enc.down{down.stride}"
            h, L = self._conv(h, B, L, down, nat.EPI_ELU if i == n - 1 else 0)
        self._tag = "enc.last"
        h, L = self._conv(h, B, L, self.enc_last)
        return h, L

    # ------------------------------------------------------------ streaming
    def stream_conv_layers(self) -> list[tuple[_Conv, str]]:
        """The convolutions a streaming encode caches, in the reference's
        order (encoder modules, then the bottleneck downsample;
        ``model.py:3047-3068``), with their padding modes."""
        convs = [(self.enc_first, "constant")]
        for (c1, c2), down in self.enc_stages:
            convs += [(c1, "constant"), (c2, "constant"), (down, "constant")]
        convs.append((self.enc_last, "constant"))
        if self.bottleneck:
            convs.append((self.down, "replicate"))
        return convs

    def _stream_conv(self, x, layer: _Conv, cache, idx: int, flags: int = 0, residual=None):
        """One cached causal conv: the layer runs on (context ++ chunk) with no
        padding; the cache keeps the newest ``k - stride`` input rows."""
        B, L, _ = x.shape
        ctx = cache.update(x, idx)
        buf = torch.cat((ctx, x), dim=1) if ctx.shape[1] else x
        total = buf.shape[1]
        if total < layer.k:
            raise RuntimeError(f"streaming chunk too short: {total} rows for a kernel of {layer.k}")
        rows = (total - layer.k) // layer.stride + 1
        y = torch.empty((B, rows, layer.c_out), device=self.device)
        self._call("fm_conv1d_valid", buf, B, total, layer.c_in, layer.w,
                   layer.b, layer.c_out, layer.k, layer.stride, flags | layer.flags, residual,
                   y, self.workspace, _WORKSPACE_BYTES)
        return y, rows

    def _encoder_seanet_stream(self, x, B, cache):
        i = 0
        self._tag = "enc.first"
        h, L = self._stream_conv(x, self.enc_first, cache, i)
        i += 1
        n = len(self.enc_stages)
        for s, ((c1, c2), down) in enumerate(self.enc_stages):
            self._tag = f"enc.res{down.c_in}"
            hid, _ = self._stream_conv(h, c1, cache, i, nat.ELU_IN | nat.EPI_ELU)
            h, L = self._stream_conv(hid, c2, cache, i + 1, nat.EPI_RES_ADD | nat.EPI_ELU, residual=h)
            self._tag = f"enc.down{down.stride}"
            h, L = self._stream_conv(h, down, cache, i + 2, nat.EPI_ELU if s == n - 1 else 0)
            i += 3
        self._tag = "enc.last"
        return self._stream_conv(h, self.enc_last, cache, i)

    def transformer_cached(self, h, B, T, layers, kv):
        """Transformer continuing from a ``MimiKVCache``: positions start at
        the cache length; each layer attends to its retained ``window - 1``
        rotated keys/values plus this chunk's (``model.py:2129-2232``)."""
        cfg = self.config
        M = B * T
        C = cfg.hidden_size
        nh, nkv, hd = cfg.num_attention_heads, cfg.num_key_value_heads, cfg.head_dim
        lib = nat.library()
        fused = (M <= _ROW_LINEAR_MAX_ROWS and hd == 64
                 and lib.fm_row_linear_supported(C, layers[0].wqkv.shape[0])
                 and lib.fm_row_linear_supported(C, layers[0].w1.shape[0])
                 and lib.fm_row_linear_supported(nh * hd, C))
        kv.configure_sliding_window(cfg.sliding_window)
        past = kv.get_seq_length()
        cos, sin = self._rope_tables(past + T)
        cos, sin = cos[past:], sin[past:]
        h = h.reshape(M, C)
        att = torch.empty((M, nh * hd), device=self.device)
        qd, kd = nh * hd, nkv * hd
        xln = None if fused else torch.empty((M, C), device=self.device)
        for li, lay in enumerate(layers):
            if fused:
                qkv = self._row_linear(h, M, lay.wqkv, ln=lay.ln1, rope=(cos, sin, qd + kd, T))
            else:
                self._call("fm_layer_norm", h, lay.ln1[0], lay.ln1[1],
                           M, C, cfg.norm_eps, xln)
                qkv = self._linear(xln, M, lay.wqkv)
                self._call("fm_apply_rope", qkv, M, qkv.shape[1], qd + kd, hd,
                           cos, sin, T)
            ld = qkv.shape[1]
            q3 = qkv.view(B, T, ld)
            keys, values = kv.update(q3[:, :, qd:qd + kd], q3[:, :, qd + kd:], li)
            n = keys.shape[1] - T
            comb = torch.empty((B, n + T, ld), device=self.device)
            comb[:, :, qd:qd + kd] = keys
            comb[:, :, qd + kd:] = values
            comb[:, n:, :qd] = q3[:, :, :qd]
            self._call("fm_window_attention_rows", comb, ld, 0, qd, qd + kd, None, None,
                       B, n + T, n, nh, nkv, hd, cfg.sliding_window, 1.0 / (hd ** 0.5),
                       att, qd)
            if fused:
                self._row_linear(att, M, lay.wo, nat.EPI_RES_SCALE, residual=h, scale=lay.ls1, out=h)
                ff = self._row_linear(h, M, lay.w1, nat.EPI_GELU, ln=lay.ln2)
            else:
                self._linear(att, M, lay.wo, nat.EPI_RES_SCALE, residual=h, scale=lay.ls1, out=h)
                self._call("fm_layer_norm", h, lay.ln2[0], lay.ln2[1],
                           M, C, cfg.norm_eps, xln)
                ff = self._linear(xln, M, lay.w1, nat.EPI_GELU)
            self._proj(ff, M, lay.w2, nat.EPI_RES_SCALE, residual=h, scale=lay.ls2, out=h)
        return h.reshape(B, T, C)

    def quantize(self, h, B, T, nq):
        cfg = self.config
        M = B * T
        vq = self.vq
        proj = self.quantizer_inputs(h, B, T)
        self._tag = "rvq.encode"
        codes = torch.empty((B, nq, T), dtype=torch.int64, device=self.device)
        ws_bytes = nat.library().fm_rvq_split_workspace_bytes(M, vq, cfg.codebook_size)
        n_sem = min(cfg.num_semantic_quantizers, nq)
        # Both chains in shared launches (step s of each branch in one grid).
        ws = torch.empty((ws_bytes + 3) // 4, device=self.device)
        self._call("fm_rvq_encode_split", proj, 2 * vq, M, T, vq, cfg.codebook_size,
                   n_sem, nq - n_sem, self.embeds, self.embeds_t,
                   self.norms, codes, nq * T, ws, ws_bytes)
        return codes

    def decode(self, codes: torch.Tensor, out_length: int | None = None, kv_cache=None) -> torch.Tensor:
        """``[B, nq, T]`` int64 codes -> ``[B, 1, out_length]`` float32 audio.
        With ``kv_cache`` the decoder transformer continues from it; everything
        else decodes the chunk alone (``model.py:3139-3170``)."""
        cfg = self.config
        B, nq, T = codes.shape
        M = B * T
        vq = self.vq
        q = torch.empty((M, 2 * vq), device=self.device)
        self._tag = "rvq.decode"
        self._call("fm_rvq_decode", codes, B, nq, T, cfg.num_semantic_quantizers,
                 self.embeds, cfg.codebook_size, vq, q)
        self._tag = "rvq.out"
        L = T
        packed = self._packed.get(self.w_out.data_ptr())
        fused_up = (self.bottleneck and self.up_k == 4 and packed is not None and M <= _ROW16_MAX_ROWS
                    and self.w_out.shape[1] == 512 and cfg.hidden_size % 32 == 0)
        if fused_up:
            # Output projection and the depthwise upsample in one launch.
            h = torch.empty((B, 2 * T, cfg.hidden_size), device=self.device)
            self._call("fm_row_linear_packed_upsample", q, M, 2 * vq, packed, cfg.hidden_size, T,
                       self.up_w, h)
            L = 2 * T
        else:
            h = self._proj(q, M, self.w_out).reshape(B, T, cfg.hidden_size)
        self._tag = "up"
        if self.bottleneck and not fused_up:
            up = torch.empty((B, L * 2, cfg.hidden_size), device=self.device)
            self._call("fm_upsample_depthwise", h, B, L, cfg.hidden_size,
                     self.up_w, self.up_k, 2, up)
            h, L = up, 2 * L
        if kv_cache is None:
            h = self.transformer(h, B, L, self.dec_tf, "dec.tf")
        else:
            h = self.transformer_cached(h, B, L, self.dec_tf, kv_cache)
        self._tag = "dec.first"
        h, L = self._conv(h, B, L, self.dec_first, nat.EPI_ELU)
        n = len(self.dec_stages)
        for i, (convt, block) in enumerate(self.dec_stages):
            self._tag = f"dec.up{convt.stride}"
            h, L = self._convt(h, B, L, convt)
            c1, c2 = block
            if i == n - 1 and self._fuse_last(block):
                # The last block feeds the waveform conv on chip.
                full = L
                out_length = full if out_length is None else min(out_length, full)
                self._tag = "dec.res64+last"
                lib = nat.library()
                d = torch.empty((lib.fm_resblock64_conv_workspace_bytes(B, L) + 3) // 4, device=self.device)
                y = torch.empty((B, out_length), device=self.device)
                last = self.dec_last
                self._call("fm_resblock64_conv", h, B, L, c1.w, c1.b,
                           c2.w, c2.b, 1 | nat.ACT_EXP | (c1.flags & c2.flags & nat.WEIGHTS_X6), last.w, last.b,
                           out_length, y, d, d.numel() * 4)
                return y.view(B, 1, out_length)
            h = self._resblock(h, B, L, block, elu_after=True, tag=f"dec.res{convt.c_out}", act_exp=True)
        full = L
        out_length = full if out_length is None else min(out_length, full)
        self._tag = "dec.last"
        y, _ = self._conv(h, B, L, self.dec_last, y_len=out_length)
        c_out = self.dec_last.c_out
        if c_out == 1:
            return y.view(B, 1, out_length)
        return y.transpose(1, 2).contiguous()

    # ------------------------------------------------------- measurement
    def layer_op(self, name: str, batch: int, samples: int):
        """A closure running one SEANet contraction at its real shape for a
        ``batch x samples`` round trip (names as in ``flops.layer_table``), on
        fixed random inputs.  Used to time a single kernel."""
        cfg = self.config
        specs = {}
        L = samples
        specs["enc.first"] = (self.enc_first, L, 0, False)
        ch = cfg.num_filters
        for i, r in enumerate(reversed(cfg.upsampling_ratios)):
            (c1, c2), down = self.enc_stages[i]
            specs[f"enc.res{ch}.c1"] = (c1, L, nat.ELU_IN | nat.EPI_ELU, False)
            specs[f"enc.res{ch}.c2"] = (c2, L, nat.EPI_RES_ADD | nat.EPI_ELU, True)
            specs[f"enc.down{r}"] = (down, L, 0, False)
            L = -(-L // r)
            ch *= 2
        specs["enc.last"] = (self.enc_last, L, 0, False)
        if self.bottleneck:
            L = 2 * (-(-L // 2))
        specs["dec.first"] = (self.dec_first, L, nat.EPI_ELU, False)
        for i, r in enumerate(cfg.upsampling_ratios):
            convt, (c1, c2) = self.dec_stages[i]
            specs[f"dec.up{r}"] = (convt, L, 0, False)
            L *= r
            ch = convt.c_out
            specs[f"dec.res{ch}.c1"] = (c1, L, nat.ELU_IN | nat.EPI_ELU, False)
            specs[f"dec.res{ch}.c2"] = (c2, L, nat.EPI_RES_ADD | nat.EPI_ELU, True)
        specs["dec.last"] = (self.dec_last, L, 0, False)
        layer, length, flags, needs_res = specs[name]
        g = torch.Generator(device=self.device).manual_seed(0)
        x = torch.randn((batch, length, layer.c_in), device=self.device, generator=g)
        if isinstance(layer, _ConvT):
            return lambda: self._convt(x, batch, length, layer)
        res = None
        if needs_res:
            res = torch.randn((batch, -(-length // layer.stride), layer.c_out), device=self.device,
                              generator=g)
        return lambda: self._conv(x, batch, length, layer, flags, residual=res)
