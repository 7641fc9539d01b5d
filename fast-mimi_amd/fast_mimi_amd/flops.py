"""Algorithmic work of one Mimi encode+decode (2 x multiply-accumulates).

Counts convolutions, transposed convolutions, GEMMs, attention (scores and
weighted sum over the causal window) and RVQ distance GEMMs; elementwise work
is excluded.  Conv: B*L_out*C_out*(C_in/g)*K; ConvT: B*L_in*C_in*(C_out/g)*K;
transformer layer: B*(4*T*h^2 + 2*T*h*ffn + 2*h*sum_t min(t+1, window));
RVQ: B*T*(2*h*vq + nq*entries*(vq+2)) encode + B*T*2*vq*h decode.
At the published config this gives 109.2 GFLOP for 10 s, B=1, nq=8.
"""

from __future__ import annotations

from .config import MimiConfig


def _layers(config: MimiConfig, batch: int, samples: int):
    """Yield (name, kind, flops, rows, k, n) per contraction, in execution order."""
    c = config
    nf = c.num_filters
    L = samples
    yield ("enc.first", "conv", 2 * batch * L * nf * c.audio_channels * c.kernel_size, batch * L,
           c.audio_channels * c.kernel_size, nf)
    ch = nf
    for ratio in reversed(c.upsampling_ratios):
        hid = ch // c.compress
        yield (f"enc.res{ch}.c1", "conv", 2 * batch * L * hid * ch * c.residual_kernel_size,
               batch * L, ch * c.residual_kernel_size, hid)
        yield (f"enc.res{ch}.c2", "conv", 2 * batch * L * ch * hid, batch * L, hid, ch)
        L = -(-L // ratio)
        yield (f"enc.down{ratio}", "conv", 2 * batch * L * 2 * ch * ch * 2 * ratio, batch * L,
               2 * ratio * ch, 2 * ch)
        ch *= 2
    yield ("enc.last", "conv", 2 * batch * L * c.hidden_size * ch * c.last_kernel_size, batch * L,
           ch * c.last_kernel_size, c.hidden_size)
    T25 = L
    yield from _transformer("enc.tf", c, batch, T25)
    T = T25
    if c.frame_rate != c.encodec_frame_rate:
        T = -(-T25 // 2)
        yield ("down", "conv", 2 * batch * T * c.hidden_size * c.hidden_size * 4, batch * T,
               4 * c.hidden_size, c.hidden_size)
    yield ("rvq.in", "gemm", 2 * batch * T * c.hidden_size * 2 * c.vector_quantization_hidden_dimension,
           batch * T, c.hidden_size, 2 * c.vector_quantization_hidden_dimension)


def _transformer(name, c: MimiConfig, batch: int, T: int):
    h = c.hidden_size
    win = sum(min(t + 1, c.sliding_window) for t in range(T))
    for i in range(c.num_hidden_layers):
        yield (f"{name}{i}.qkv", "gemm", 2 * batch * T * h * 3 * h, batch * T, h, 3 * h)
        yield (f"{name}{i}.attn", "attn", 2 * 2 * batch * h * win, batch * T, 0, 0)
        yield (f"{name}{i}.o", "gemm", 2 * batch * T * h * h, batch * T, h, h)
        yield (f"{name}{i}.fc1", "gemm", 2 * batch * T * h * c.intermediate_size, batch * T, h,
               c.intermediate_size)
        yield (f"{name}{i}.fc2", "gemm", 2 * batch * T * h * c.intermediate_size, batch * T,
               c.intermediate_size, h)


def _decode_layers(config: MimiConfig, batch: int, frames: int):
    c = config
    vq = c.vector_quantization_hidden_dimension
    yield ("rvq.out", "gemm", 2 * batch * frames * 2 * vq * c.hidden_size, batch * frames, 2 * vq,
           c.hidden_size)
    T = frames
    if c.frame_rate != c.encodec_frame_rate:
        yield ("up", "dw", 2 * batch * T * c.hidden_size * 4, batch * T, 0, 0)
        T *= 2
    yield from _transformer("dec.tf", c, batch, T)
    ch = nf_top = c.num_filters * 2 ** len(c.upsampling_ratios)
    yield ("dec.first", "conv", 2 * batch * T * ch * c.hidden_size * c.kernel_size, batch * T,
           c.hidden_size * c.kernel_size, ch)
    L = T
    for ratio in c.upsampling_ratios:
        yield (f"dec.up{ratio}", "convt", 2 * batch * L * ch * (ch // 2) * 2 * ratio, batch * L,
               2 * ch, ratio * ch // 2)
        L *= ratio
        ch //= 2
        hid = ch // c.compress
        yield (f"dec.res{ch}.c1", "conv", 2 * batch * L * hid * ch * c.residual_kernel_size,
               batch * L, ch * c.residual_kernel_size, hid)
        yield (f"dec.res{ch}.c2", "conv", 2 * batch * L * ch * hid, batch * L, hid, ch)
    yield ("dec.last", "conv", 2 * batch * L * c.audio_channels * ch * c.last_kernel_size,
           batch * L, ch * c.last_kernel_size, c.audio_channels)
    del nf_top


def layer_table(config: MimiConfig, batch: int, samples: int, num_quantizers: int):
    rows = list(_layers(config, batch, samples))
    frames = rows[-1][3] // batch
    vq = config.vector_quantization_hidden_dimension
    rows.append(("rvq.dist", "rvq", 2 * batch * frames * num_quantizers * config.codebook_size * (vq + 2),
                 batch * frames, vq + 2, config.codebook_size))
    rows.extend(_decode_layers(config, batch, frames))
    return rows


def roundtrip_flops(config: MimiConfig, batch: int, samples: int, num_quantizers: int) -> int:
    return sum(r[2] for r in layer_table(config, batch, samples, num_quantizers))
