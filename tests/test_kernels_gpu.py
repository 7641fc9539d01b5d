"""Per-kernel parity of the HIP library against float64 CPU references.

Every call goes through the C ABI (``fast_mimi_amd._native``) with device
pointers.  Floating-point kernels are held to FP32 accumulation error against
a float64 evaluation of the same formula (the oracle's op definitions); the
RVQ gather-sum and argmin are held to exact equality (near-ties excepted and
reported for the argmin).
"""

from __future__ import annotations

import math

import numpy as np

import pytest
import torch
import torch.nn.functional as F

from fast_mimi_amd import _native as nat
from fast_mimi_amd.runtime import _Conv, _ConvT, rope_tables
from fast_mimi_amd.config import MimiConfig
from oracle.mimi_oracle import causal_conv1d, causal_conv_transpose1d, MimiOracle
from rvq_check import check_codes, reference_rvq_rows

pytestmark = pytest.mark.gpu
DEV = "cuda"
WS_BYTES = 64 << 20


@pytest.fixture(scope="module")
def ws():
    return torch.empty(WS_BYTES // 4, device=DEV)


def stream():
    return torch.cuda.current_stream().cuda_stream


def close(got, want, rel=2e-5):
    """FP32-accumulation bound against a float64 result."""
    got = got.double().cpu()
    want = want.double().cpu()
    scale = want.abs().max().item() + 1e-30
    err = (got - want).abs().max().item()
    assert err <= rel * scale, f"max err {err:.3e} vs scale {scale:.3e}"


def close_dot(got, want, absref, rel=1e-5):
    """Per-element FP32 accumulation bound: |got - want| <= rel * sum_k |a_k b_k|
    (absref, the same contraction on absolute values in float64), so
    small-magnitude outputs are held as tightly as large ones."""
    got = got.double().cpu()
    want = want.double().cpu()
    absref = absref.double().cpu()
    err = (got - want).abs()
    bound = rel * absref + 1e-30
    worst = (err / bound).max().item()
    assert worst <= 1.0, f"error {worst:.2f}x the per-element bound (rel {rel:.0e} of sum |a b|)"


def with_planes(w):
    """A packed weight W^T [N, K] followed by its bf16x6 planes
    (fm_split_weights, k16-tile order [3][K/16][N][16]), as the runtime
    stores it; returns the FP32 view at the buffer's start."""
    rows, cols = w.shape
    if cols % 16:
        pytest.skip("bf16x6 planes need K to be a multiple of 16")
    n = w.numel()
    buf = torch.empty(n + 3 * n // 2, device=DEV)
    buf[:n].copy_(w.reshape(-1))
    nat.call("fm_split_weights", buf.data_ptr(), rows, cols, buf.data_ptr() + 4 * n, stream())
    torch.cuda.synchronize()
    return buf[:n].view(w.shape)


def planes_of(buf):
    """The three planes after a with_planes weight, back in [3][N][K] order."""
    rows, cols = buf.shape
    n = buf.numel()
    raw = torch.empty(0, dtype=torch.bfloat16, device=DEV).set_(
        buf.reshape(-1).untyped_storage(), n * 2, (3, cols // 16, rows, 16))
    return raw.permute(0, 2, 1, 3).reshape(3, rows, cols)


def test_split_weights_pieces_sum_to_the_weight():
    """Each float is three round-to-nearest bf16 pieces whose sum is within
    2^-24 of it, each piece at most half an ulp of the previous remainder;
    the planes are in k16-tile order."""
    g = torch.Generator().manual_seed(3)
    w = (torch.randn(48 * 80, generator=g) * torch.logspace(-6, 3, 48 * 80)).view(48, 80).to(DEV)
    buf = with_planes(w)
    raw = planes_of(buf)
    h = raw.float().cpu().double()
    wd = w.cpu().double()
    assert torch.equal(raw[0].cpu(), w.cpu().to(torch.bfloat16))
    assert torch.equal(raw[1].cpu(), (wd - h[0]).float().to(torch.bfloat16))
    assert torch.all((wd - h.sum(0)).abs() <= wd.abs() * 2.0 ** -24)
    with pytest.raises(nat.NativeError, match="bad argument"):
        nat.call("fm_split_weights", buf.data_ptr(), 0, 16, buf.data_ptr(), stream())
    with pytest.raises(nat.NativeError, match="unsupported"):
        nat.call("fm_split_weights", buf.data_ptr(), 4, 24, buf.data_ptr(), stream())


def run_conv(x_ncl, w, b, stride, pad_mode, flags, ws, residual_ncl=None, y_len=None, x6=False):
    B, C, L = x_ncl.shape
    layer = _Conv(w.to(DEV), None if b is None else b.to(DEV), stride, pad_mode)
    if x6:
        layer.w, flags = with_planes(layer.w), flags | nat.WEIGHTS_X6
    x = x_ncl.transpose(1, 2).contiguous().to(DEV)
    rows = -(-L // stride)
    y_len = rows if y_len is None else y_len
    y = torch.empty((B, y_len, layer.c_out), device=DEV)
    res = None if residual_ncl is None else residual_ncl.transpose(1, 2).contiguous().to(DEV)
    nat.call("fm_conv1d", x.data_ptr(), B, L, C, layer.w.data_ptr(),
             None if layer.b is None else layer.b.data_ptr(), layer.c_out, layer.k, stride,
             layer.replicate, flags, None if res is None else res.data_ptr(), y.data_ptr(), y_len,
             ws.data_ptr(), WS_BYTES, stream())
    torch.cuda.synchronize()
    return y.cpu().transpose(1, 2)


CONV_CASES = [
    # B, Cin, Cout, k, stride, L
    (1, 1, 64, 7, 1, 1000),
    (2, 64, 32, 3, 1, 777),
    (1, 32, 64, 1, 1, 513),
    (2, 64, 128, 8, 4, 1001),
    (1, 128, 256, 10, 5, 303),
    (1, 256, 512, 12, 6, 121),
    (1, 512, 1024, 16, 8, 250),     # split-K path (small M, K = 8192)
    (1, 1024, 512, 3, 1, 250),
    (3, 64, 1, 3, 1, 999),          # Cout = 1
    (2, 2, 4, 4, 2, 9),             # tiny channels, scalar loads
    (1, 4, 2, 3, 1, 1),             # length 1
    (1, 16, 16, 4, 2, 5),
    (1, 64, 32, 3, 1, 140000),     # 256x32 tiles
    (1, 32, 64, 1, 1, 70000),      # 128x64 tiles
    (1, 64, 256, 4, 2, 70000),     # 128x128 tiles
    (1, 64, 128, 8, 4, 240000),    # 256x128 tiles
    (1, 64, 64, 3, 1, 60000),      # 256x64 tiles
    (2, 128, 256, 10, 5, 300000),  # 256x256 tiles, batch seam inside a tile
    (1, 256, 512, 12, 6, 12000),   # 256x64 tiles split along K (M = 2000, K = 3072)
    (1, 512, 1024, 16, 8, 2000),   # 64x64 16x16-MFMA tiles split along K (M = 250)
    (2, 512, 256, 3, 1, 300),      # 64x64 16x16-MFMA tiles, batch seam inside a tile
    (1, 512, 512, 4, 2, 250),      # 32x32 tiles, K split inside the block and across blocks
    (3, 1024, 96, 2, 1, 70),       # 32x32 tiles, partial column tile
]


@pytest.mark.parametrize("B,cin,cout,k,stride,L", CONV_CASES)
def test_conv1d(B, cin, cout, k, stride, L, ws):
    g = torch.Generator().manual_seed(B * 1000 + cin + cout + k + L)
    x = torch.randn(B, cin, L, generator=g)
    w = torch.randn(cout, cin, k, generator=g) / math.sqrt(cin * k)
    b = torch.randn(cout, generator=g) * 0.1
    got = run_conv(x, w, b, stride, "constant", 0, ws)
    want = causal_conv1d(x.double(), w.double(), b.double(), stride)
    assert got.shape == want.shape
    close(got, want)
    close_dot(got, want, causal_conv1d(x.double().abs(), w.double().abs(), b.double().abs(), stride))


# Direct-load tiles (C_in a multiple of 16, zero padding, no ELU on load):
# 128x128 with a partial column tile and an odd row count, the 192x128 and
# 64x128 picks of few-hundred-tile shapes, and a K-split one.
DL_CASES = [
    # B, Cin, Cout, k, stride, L, y_len
    (1, 64, 160, 4, 2, 70001, None),
    (2, 48, 132, 2, 1, 40003, 39000),
    (1, 512, 1536, 1, 1, 4000, None),
    (1, 512, 512, 1, 1, 4000, 3999),
    (16, 512, 512, 1, 1, 250, None),
    (1, 256, 512, 12, 6, 12003, None),
    (1, 2048, 512, 1, 1, 4000, None),   # long K, one 64x128 tile per CU, unsplit
    (1, 480, 512, 1, 1, 4000, None),    # 64x128 pick with C_in % 64 == 32 (32-deep tile)
    (1, 128, 256, 8, 4, 240001, 59990),  # >= 384 256x128 bf16x6 tiles, partial last row tile, crop
    (1, 512, 1536, 1, 1, 2500, None),   # 240 128x128 tiles: 64x128 bf16x6 tiles
    (1, 2048, 512, 1, 1, 2500, 2499),   # long K, 80 tiles: 64x128 bf16x6 tiles split along K
    (1, 128, 1024, 3, 1, 5000, 4990),   # 320 128x128 tiles: 192x128 bf16x6 tiles, partial, crop
    (1, 256, 1024, 8, 1, 2500, None),   # 160 128x128 tiles, K 2048: bf16x6 split in two
    (4, 64, 256, 4, 1, 6000, 2000),     # crop to a third: tiles span dropped rows and clip seams
]


@pytest.mark.parametrize("B,cin,cout,k,stride,L,y_len", DL_CASES)
@pytest.mark.parametrize("epi", ["plain", "res_elu"])
@pytest.mark.parametrize("x6", [False, True], ids=["fp32", "bf16x6"])
def test_conv1d_direct_load_tiles(B, cin, cout, k, stride, L, y_len, epi, x6, ws):
    g = torch.Generator().manual_seed(B * 31 + cin + cout + k + L)
    x = torch.randn(B, cin, L, generator=g)
    w = torch.randn(cout, cin, k, generator=g) / math.sqrt(cin * k)
    b = torch.randn(cout, generator=g) * 0.1
    rows = -(-L // stride)
    want = causal_conv1d(x.double(), w.double(), b.double(), stride)
    if epi == "plain":
        got = run_conv(x, w, b, stride, "constant", 0, ws, y_len=y_len, x6=x6)
        absref = causal_conv1d(x.double().abs(), w.double().abs(), b.double().abs(), stride)
        absref = absref[..., :y_len] if y_len is not None else absref
        close_dot(got, want[..., :y_len] if y_len is not None else want, absref)
    else:
        res = torch.randn(B, cout, rows, generator=g)
        got = run_conv(x, w, b, stride, "constant", nat.EPI_RES_ADD | nat.EPI_ELU, ws,
                       residual_ncl=res, y_len=y_len, x6=x6)
        want = F.elu(res.double() + want)
    want = want[..., :y_len] if y_len is not None else want
    assert got.shape == want.shape
    close(got, want)


def _random_x6_cases(n, seed=11):
    """Seeded conv shapes large enough for the bf16x6 tiles (>= 192 tiles of
    128 x 128 counting splits), with crops, residual epilogues, batch seams,
    partial row and column tiles."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        B = int(rng.integers(1, 4))
        cin = int(rng.choice([16, 32, 48, 64, 96, 128]))
        cout = 4 * int(rng.integers(32, 160))
        k = int(rng.integers(1, 9))
        stride = int(rng.integers(1, k + 1))
        rows = int(rng.integers(8000, 30000)) // B
        L = rows * stride - int(rng.integers(0, stride))
        rows = -(-L // stride)
        if B * rows * cout < 192 * 128 * 128:
            continue
        y_len = None if rng.random() < 0.5 else int(rng.integers(rows // 2, rows + 1))
        epi = "plain" if rng.random() < 0.5 else "res_elu"
        out.append((B, cin, cout, k, stride, L, y_len, epi))
    return out


@pytest.mark.parametrize("B,cin,cout,k,stride,L,y_len,epi", _random_x6_cases(12))
def test_conv1d_bf16x6_random_shapes(B, cin, cout, k, stride, L, y_len, epi, ws):
    """Randomised shapes through the bf16x6 tiles (register epilogue: buffer
    stores over a tile's rows, crop remap, residual loads) against float64."""
    g = torch.Generator().manual_seed(B * 7 + cin + cout + k + L)
    x = torch.randn(B, cin, L, generator=g)
    w = torch.randn(cout, cin, k, generator=g) / math.sqrt(cin * k)
    b = torch.randn(cout, generator=g) * 0.1
    rows = -(-L // stride)
    want = causal_conv1d(x.double(), w.double(), b.double(), stride)
    if epi == "plain":
        got = run_conv(x, w, b, stride, "constant", 0, ws, y_len=y_len, x6=True)
    else:
        res = torch.randn(B, cout, rows, generator=g)
        got = run_conv(x, w, b, stride, "constant", nat.EPI_RES_ADD | nat.EPI_ELU, ws,
                       residual_ncl=res, y_len=y_len, x6=True)
        want = F.elu(res.double() + want)
    assert "x6d" in nat.last_gemm_plan(), nat.last_gemm_plan()
    want = want[..., :y_len] if y_len is not None else want
    assert got.shape == want.shape
    close(got, want)


def test_bf16x6_large_input_loads_agree(ws):
    """The direct-load bf16x6 tiles read A through a buffer resource when the
    input is below 2 GiB and through global addresses above it: a 2.3 GiB
    two-clip input (global path) must give, for its second clip, exactly the
    output of that clip alone (buffer path), causal edge included."""
    B, cin, cout, k, stride = 2, 64, 128, 8, 4
    L = 4_500_000  # 1.15 GB of channels-last input per clip
    g = torch.Generator(device=DEV).manual_seed(5)
    x = torch.randn(B, L, cin, device=DEV, generator=g)
    w = torch.randn(cout, cin, k, generator=torch.Generator().manual_seed(6)) / math.sqrt(cin * k)
    layer = _Conv(w.to(DEV), None, stride, "constant")
    wx = with_planes(layer.w)
    rows = -(-L // stride)
    outs = []
    for xb, bb in ((x, B), (x[1:].contiguous(), 1)):
        y = torch.empty((bb, rows, cout), device=DEV)
        nat.call("fm_conv1d", xb.data_ptr(), bb, L, cin, wx.data_ptr(), None, cout, k, stride, 0,
                 nat.WEIGHTS_X6, None, y.data_ptr(), rows, ws.data_ptr(), WS_BYTES, stream())
        torch.cuda.synchronize()
        outs.append(y[-1].clone())
        del y
    assert torch.equal(outs[0], outs[1])
    # A few rows against float64 (the causal edge and an interior window):
    # y[t] = sum_j W[:, :, j] x[t * stride - (k - stride) + j], zero outside.
    wd = w.double()
    for t in (0, 1, rows // 2):
        idx = torch.arange(k) + t * stride - (k - stride)
        xs = x[1, idx.clamp(0, L - 1)].double().cpu() * ((idx >= 0) & (idx < L)).double()[:, None]
        want = torch.einsum("jc,ocj->o", xs, wd)
        close(outs[1][t].cpu()[None], want[None])


@pytest.mark.parametrize("B,cin,cout,L", [(1, 512, 256, 2000), (16, 512, 256, 2000), (2, 256, 128, 9001),
                                          (1, 128, 1024, 5000), (1, 512, 256, 16500)])
def test_conv1d_bf16x6_elu_on_load(B, cin, cout, L, ws):
    """bf16x6 tiles with ELU applied to the A operand as it is loaded (the
    residual block's first conv, k = 3), ELU epilogue, vs float64."""
    g = torch.Generator().manual_seed(B + cin + L)
    x = torch.randn(B, cin, L, generator=g)
    w = torch.randn(cout, cin, 3, generator=g) / math.sqrt(cin * 3)
    b = torch.randn(cout, generator=g) * 0.1
    got = run_conv(x, w, b, 1, "constant", nat.ELU_IN | nat.EPI_ELU, ws, x6=True)
    want = F.elu(causal_conv1d(F.elu(x.double()), w.double(), b.double(), 1))
    close(got, want)


@pytest.mark.parametrize("B,L,y_len", [(1, 1, 1), (2, 2, 2), (1, 62, 62), (2, 63, 60), (3, 999, 999),
                                       (1, 240000, 240000), (2, 24001, 23995)])
@pytest.mark.parametrize("elu_in", [0, 1])
def test_conv1d_single_output_channel(B, L, y_len, elu_in, ws):
    """The waveform layer (64 -> 1, k = 3): ELU on load, crop, block seams."""
    g = torch.Generator().manual_seed(B * 7 + L + y_len)
    x = torch.randn(B, 64, L, generator=g)
    w = torch.randn(1, 64, 3, generator=g) / 8
    b = torch.randn(1, generator=g) * 0.1
    got = run_conv(x, w, b, 1, "constant", nat.ELU_IN if elu_in else 0, ws, y_len=y_len)
    xin = F.elu(x.double()) if elu_in else x.double()
    want = causal_conv1d(xin, w.double(), b.double())[..., :y_len]
    assert got.shape == want.shape
    close(got, want)


@pytest.mark.parametrize("B,L", [(1, 250), (2, 7), (1, 1), (3, 64)])
def test_conv1d_replicate(B, L, ws):
    g = torch.Generator().manual_seed(L)
    x = torch.randn(B, 64, L, generator=g)
    w = torch.randn(64, 64, 4, generator=g) / 16
    got = run_conv(x, w, None, 2, "replicate", 0, ws)
    want = causal_conv1d(x.double(), w.double(), None, 2, pad_mode="replicate")
    close(got, want)


# Few-row long-K convolutions (fm_conv1d_rows): the encoder's last conv
# (1024 -> 512 k3), the replicate-padded downsample (512 -> 512 k4 s2, odd
# and even lengths) and the decoder's first conv (512 -> 1024 k7), with batch
# seams and partial 16-row blocks; same float64 bars as fm_conv1d, and the
# same result as fm_conv1d to FP32 accumulation error.
ROWCONV_CASES = [
    # B, Cin, Cout, k, stride, L, pad_mode, flags
    (1, 1024, 512, 3, 1, 250, "constant", 0),
    (1, 1024, 512, 3, 1, 250, "constant", nat.ELU_IN | nat.EPI_ELU),
    (1, 512, 512, 4, 2, 250, "replicate", 0),
    (2, 512, 512, 4, 2, 63, "replicate", 0),
    (3, 512, 512, 4, 2, 1, "replicate", 0),
    (1, 512, 1024, 7, 1, 250, "constant", nat.EPI_ELU),
    (2, 512, 1024, 7, 1, 37, "constant", 0),
    (2, 256, 512, 12, 1, 70, "constant", nat.ELU_IN),  # 3072-deep with k = 12 taps of 256
    (1, 512, 256, 3, 1, 2000, "constant", nat.ELU_IN | nat.EPI_ELU),  # residual block k3 conv, 2000 rows
    (1, 256, 512, 1, 1, 2000, "constant", nat.EPI_RES_ADD | nat.EPI_ELU),  # its 1x1 conv (bf16x6 only)
    (2, 256, 512, 1, 1, 77, "constant", nat.EPI_RES_ADD),
]


@pytest.mark.parametrize("x6", [False, True], ids=["fp32", "bf16x6"])
@pytest.mark.parametrize("B,cin,cout,k,stride,L,pad_mode,flags", ROWCONV_CASES)
def test_conv1d_rows(B, cin, cout, k, stride, L, pad_mode, flags, x6, ws):
    lib = nat.library()
    if not lib.fm_conv1d_rows_supported(cin, cout, k, nat.WEIGHTS_X6 if x6 else 0):
        assert not x6 and cin * k == 256
        pytest.skip("256-deep convs run only on the bf16x6 weights")
    g = torch.Generator().manual_seed(B * 7 + cin + cout + k + L)
    x = torch.randn(B, cin, L, generator=g)
    w = torch.randn(cout, cin, k, generator=g) / math.sqrt(cin * k)
    b = torch.randn(cout, generator=g) * 0.1 if pad_mode == "constant" else None
    layer = _Conv(w.to(DEV), None if b is None else b.to(DEV), stride, pad_mode)
    if x6:
        wr, f = with_planes(layer.w), flags | nat.WEIGHTS_X6
    else:
        wr, f = torch.empty_like(layer.w), flags
        nat.call("fm_pack_row_weights", layer.w.data_ptr(), cout, k * cin, wr.data_ptr(), stream())
    xd = x.transpose(1, 2).contiguous().to(DEV)
    rows = -(-L // stride)
    y = torch.full((B, rows, cout), float("nan"), device=DEV)
    res = torch.randn(B, cout, rows, generator=g) if flags & nat.EPI_RES_ADD else None
    resd = None if res is None else res.transpose(1, 2).contiguous().to(DEV)
    nat.call("fm_conv1d_rows", xd.data_ptr(), B, L, cin, wr.data_ptr(),
             None if layer.b is None else layer.b.data_ptr(), cout, cout, k, stride, layer.replicate, f,
             None if resd is None else resd.data_ptr(), y.data_ptr(), stream())
    torch.cuda.synchronize()
    got = y.cpu().transpose(1, 2)
    xi = F.elu(x.double()) if flags & nat.ELU_IN else x.double()
    bd = None if b is None else b.double()
    want = causal_conv1d(xi, w.double(), bd, stride, pad_mode=pad_mode)
    absref = causal_conv1d(xi.abs(), w.double().abs(), None if bd is None else bd.abs(), stride,
                           pad_mode=pad_mode)
    if res is not None:
        want = want + res.double()
    if flags & nat.EPI_ELU:
        want = F.elu(want)
    elif res is None:
        close_dot(got, want, absref)
    close(got, want)
    same = run_conv(x, w, b, stride, pad_mode, flags, ws, residual_ncl=res)
    close(got, same.double())


@pytest.mark.parametrize("B,L", [(1, 250), (2, 37)])
def test_conv_transpose1d_rows(B, L):
    """The decoder's first transposed conv (1024 -> 512, k16 s8) as the few-row
    conv over its two taps with the phase-major weight and bias period c_out."""
    g = torch.Generator().manual_seed(B + L)
    cin, cout, k, s = 1024, 512, 16, 8
    x = torch.randn(B, cin, L, generator=g)
    w = torch.randn(cin, cout, k, generator=g) / math.sqrt(cin * k / s)
    b = torch.randn(cout, generator=g) * 0.1
    layer = _ConvT(w.to(DEV), b.to(DEV), s)
    wx = with_planes(layer.w)
    xd = x.transpose(1, 2).contiguous().to(DEV)
    y = torch.full((B, L * s, cout), float("nan"), device=DEV)
    nat.call("fm_conv1d_rows", xd.data_ptr(), B, L, cin, wx.data_ptr(), layer.b.data_ptr(), cout,
             s * cout, k // s, 1, 0, nat.WEIGHTS_X6, None, y.data_ptr(), stream())
    torch.cuda.synchronize()
    got = y.cpu().transpose(1, 2)
    want = causal_conv_transpose1d(x.double(), w.double(), b.double(), s)
    close(got, want)
    close_dot(got, want, causal_conv_transpose1d(x.double().abs(), w.double().abs(), b.double().abs(), s))


def test_conv1d_rows_rejects():
    with pytest.raises(nat.NativeError, match="unsupported"):
        nat.call("fm_conv1d_rows", 1, 1, 4, 64, 1, None, 32, 32, 3, 1, 0, 0, None, 1, stream())  # K = 192
    with pytest.raises(nat.NativeError, match="unsupported"):
        nat.call("fm_conv1d_rows", 1, 1, 4, 512, 1, None, 512, 512, 4, 2, 0, nat.EPI_GELU, None, 1, stream())
    with pytest.raises(nat.NativeError, match="unsupported"):  # K = 8192
        nat.call("fm_conv1d_rows", 1, 1, 4, 512, 1, None, 1024, 1024, 16, 8, 0, nat.WEIGHTS_X6, None, 1, stream())
    with pytest.raises(nat.NativeError, match="unsupported"):  # C_in = 96: 64-deep pieces would cross taps
        nat.call("fm_conv1d_rows", 1, 1, 4, 96, 1, None, 512, 512, 32, 1, 0, 0, None, 1, stream())
    with pytest.raises(nat.NativeError, match="bad argument"):
        nat.call("fm_conv1d_rows", 1, 1, 4, 512, 1, None, 512, 512, 4, 2, 2, 0, None, 1, stream())
    with pytest.raises(nat.NativeError, match="bad argument"):  # residual epilogue without residual
        nat.call("fm_conv1d_rows", 1, 1, 4, 512, 1, None, 512, 512, 4, 2, 0, nat.EPI_RES_ADD, None, 1, stream())


def test_conv1d_fused_resblock_epilogues(ws):
    """ELU-on-load + k3 conv + ELU, then 1x1 conv + residual add + ELU."""
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 64, 300, generator=g)
    w1 = torch.randn(32, 64, 3, generator=g) / 14
    b1 = torch.randn(32, generator=g) * 0.1
    w2 = torch.randn(64, 32, 1, generator=g) / 6
    b2 = torch.randn(64, generator=g) * 0.1
    h = run_conv(x, w1, b1, 1, "constant", nat.ELU_IN | nat.EPI_ELU, ws)
    xd = x.double()
    want_h = F.elu(causal_conv1d(F.elu(xd), w1.double(), b1.double()))
    close(h, want_h)
    y = run_conv(h.contiguous(), w2, b2, 1, "constant", nat.EPI_RES_ADD | nat.EPI_ELU, ws, residual_ncl=x)
    want = F.elu(xd + causal_conv1d(want_h, w2.double(), b2.double()))
    close(y, want, rel=5e-5)


@pytest.mark.parametrize("B,C,L", [(1, 512, 2000), (1, 512, 250), (2, 512, 61)])
def test_long_k_epilogues(B, C, L, ws):
    """ELU-on-load / ELU / residual epilogues and replicate padding on the
    long-K paths (split 256x64 tiles at 2000 rows, 16x16-MFMA tiles below)."""
    g = torch.Generator().manual_seed(B * C + L)
    x = torch.randn(B, C, L, generator=g)
    w1 = torch.randn(C // 2, C, 3, generator=g) / math.sqrt(3 * C)
    b1 = torch.randn(C // 2, generator=g) * 0.1
    w2 = torch.randn(C, C // 2, 3, generator=g) / math.sqrt(1.5 * C)
    b2 = torch.randn(C, generator=g) * 0.1
    xd = x.double()
    h = run_conv(x, w1, b1, 1, "constant", nat.ELU_IN | nat.EPI_ELU, ws)
    want_h = F.elu(causal_conv1d(F.elu(xd), w1.double(), b1.double()))
    close(h, want_h)
    y = run_conv(h.contiguous(), w2, b2, 1, "constant", nat.EPI_RES_ADD | nat.EPI_ELU, ws,
                 residual_ncl=x)
    close(y, F.elu(xd + causal_conv1d(want_h, w2.double(), b2.double())), rel=5e-5)
    wr = torch.randn(C, C, 4, generator=g) / math.sqrt(4 * C)
    got = run_conv(x, wr, None, 2, "replicate", 0, ws)
    close(got, causal_conv1d(xd, wr.double(), None, 2, pad_mode="replicate"))


@pytest.mark.parametrize("B,C,L", [(1, 64, 1000), (2, 64, 129), (1, 128, 777), (3, 128, 1),
                                   (1, 256, 300), (2, 256, 33), (1, 64, 240000), (2, 128, 6001),
                                   (2, 256, 12001)])
@pytest.mark.parametrize("elu_out", [1, 0])
@pytest.mark.parametrize("x6", [False, True, "act_exp"])
def test_fused_resblock(B, C, L, elu_out, x6):
    """fm_resblock equals the reference block x + conv1x1(ELU(conv_k3(ELU(x)))),
    on FP32 weights, on weights followed by their bf16x6 planes, and with the
    e^x - 1 ELUs of FM_ACT_EXP (same bar: their error is absolute, ~1e-7)."""
    g = torch.Generator().manual_seed(C + L)
    x = torch.randn(B, C, L, generator=g)
    w1 = torch.randn(C // 2, C, 3, generator=g) / math.sqrt(3 * C)
    b1 = torch.randn(C // 2, generator=g) * 0.1
    w2 = torch.randn(C, C // 2, 1, generator=g) / math.sqrt(C // 2)
    b2 = torch.randn(C, generator=g) * 0.1
    c1, c2 = _Conv(w1.to(DEV), b1.to(DEV)), _Conv(w2.to(DEV), b2.to(DEV))
    flags = elu_out
    if x6:
        c1.w, c2.w = with_planes(c1.w), with_planes(c2.w)
        flags |= nat.WEIGHTS_X6 | (nat.ACT_EXP if x6 == "act_exp" else 0)
    xd = x.transpose(1, 2).contiguous().to(DEV)
    y = torch.empty_like(xd)
    nat.call("fm_resblock", xd.data_ptr(), B, L, C, c1.w.data_ptr(), c1.b.data_ptr(), c2.w.data_ptr(),
             c2.b.data_ptr(), flags, y.data_ptr(), stream())
    torch.cuda.synchronize()
    xd64 = x.double()
    h = F.elu(causal_conv1d(F.elu(xd64), w1.double(), b1.double()))
    want = xd64 + causal_conv1d(h, w2.double(), b2.double())
    if elu_out:
        want = F.elu(want)
    close(y.cpu().transpose(1, 2), want, rel=5e-5)


@pytest.mark.parametrize("B,L", [(1, 240000), (2, 1001), (1, 1), (3, 33), (1, 31), (2, 32), (1, 70000)])
@pytest.mark.parametrize("elu_out", [1, 0])
@pytest.mark.parametrize("x6", [False, True, "act_exp"], ids=["fp32", "bf16x6", "act_exp"])
def test_conv_resblock64_equals_conv_then_block(B, L, elu_out, x6, ws):
    """fm_conv_resblock64 == fm_conv1d (1 -> 64, k 7) then fm_resblock, bit for
    bit, on FP32 weights and on weights with their bf16x6 planes (with and
    without FM_ACT_EXP on both calls)."""
    g = torch.Generator().manual_seed(B * 31 + L)
    wav = torch.randn(B, 1, L, generator=g) * 0.5
    w0 = torch.randn(64, 1, 7, generator=g) / 3
    b0 = torch.randn(64, generator=g) * 0.1
    w1 = torch.randn(32, 64, 3, generator=g) / math.sqrt(192)
    b1 = torch.randn(32, generator=g) * 0.1
    w2 = torch.randn(64, 32, 1, generator=g) / math.sqrt(32)
    b2 = torch.randn(64, generator=g) * 0.1
    c0 = _Conv(w0.to(DEV), b0.to(DEV))
    c1, c2 = _Conv(w1.to(DEV), b1.to(DEV)), _Conv(w2.to(DEV), b2.to(DEV))
    flags = elu_out
    if x6:
        c1.w, c2.w = with_planes(c1.w), with_planes(c2.w)
        flags |= nat.WEIGHTS_X6 | (nat.ACT_EXP if x6 == "act_exp" else 0)
    wd = wav.reshape(B, L).contiguous().to(DEV)
    h = torch.empty(B, L, 64, device=DEV)
    nat.call("fm_conv1d", wd.data_ptr(), B, L, 1, c0.w.data_ptr(), c0.b.data_ptr(), 64, 7, 1, 0, 0,
             None, h.data_ptr(), L, ws.data_ptr(), WS_BYTES, stream())
    want = torch.empty_like(h)
    nat.call("fm_resblock", h.data_ptr(), B, L, 64, c1.w.data_ptr(), c1.b.data_ptr(), c2.w.data_ptr(),
             c2.b.data_ptr(), flags, want.data_ptr(), stream())
    got = torch.full_like(h, float("nan"))
    nat.call("fm_conv_resblock64", wd.data_ptr(), B, L, c0.w.data_ptr(), c0.b.data_ptr(),
             c1.w.data_ptr(), c1.b.data_ptr(), c2.w.data_ptr(), c2.b.data_ptr(), flags,
             got.data_ptr(), stream())
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    if L <= 2000:  # and against the float64 reference of the two layers
        x64 = causal_conv1d(wav.double(), w0.double(), b0.double())
        hid = F.elu(causal_conv1d(F.elu(x64), w1.double(), b1.double()))
        ref = x64 + causal_conv1d(hid, w2.double(), b2.double())
        if elu_out:
            ref = F.elu(ref)
        close(got.cpu().transpose(1, 2), ref, rel=5e-5)


@pytest.mark.parametrize("B,L,y_len", [(1, 240000, 240000), (2, 1001, 990), (1, 1, 1), (3, 33, 33),
                                       (1, 31, 2), (2, 32, 32), (1, 70000, 69999)])
@pytest.mark.parametrize("x6", [False, True, "act_exp"], ids=["fp32", "bf16x6", "act_exp"])
def test_resblock64_conv_matches_reference(B, L, y_len, x6):
    """fm_resblock64_conv == block (ELU after) then the 64 -> 1, k = 3 conv,
    cropped; the bf16x6 form (with the exact ELU, and with the e^x - 1 ELU of
    FM_ACT_EXP that the decoder uses) also against the FP32 form at every
    size."""
    g = torch.Generator().manual_seed(B * 17 + L + y_len)
    x = torch.randn(B, 64, L, generator=g)
    w1 = torch.randn(32, 64, 3, generator=g) / math.sqrt(192)
    b1 = torch.randn(32, generator=g) * 0.1
    w2 = torch.randn(64, 32, 1, generator=g) / math.sqrt(32)
    b2 = torch.randn(64, generator=g) * 0.1
    w3 = torch.randn(1, 64, 3, generator=g) / 8
    b3 = torch.randn(1, generator=g) * 0.1
    c1, c2, c3 = _Conv(w1.to(DEV), b1.to(DEV)), _Conv(w2.to(DEV), b2.to(DEV)), _Conv(w3.to(DEV), b3.to(DEV))
    xd = x.transpose(1, 2).contiguous().to(DEV)
    lib = nat.library()
    wsb = lib.fm_resblock64_conv_workspace_bytes(B, L)
    d = torch.empty((wsb + 3) // 4, device=DEV)
    out = torch.full((B, y_len), float("nan"), device=DEV)
    nat.call("fm_resblock64_conv", xd.data_ptr(), B, L, c1.w.data_ptr(), c1.b.data_ptr(), c2.w.data_ptr(),
             c2.b.data_ptr(), 1, c3.w.data_ptr(), c3.b.data_ptr(), y_len, out.data_ptr(), d.data_ptr(),
             wsb, stream())
    if x6:
        fp32 = out.clone()
        c1.w, c2.w = with_planes(c1.w), with_planes(c2.w)
        out.fill_(float("nan"))
        nat.call("fm_resblock64_conv", xd.data_ptr(), B, L, c1.w.data_ptr(), c1.b.data_ptr(), c2.w.data_ptr(),
                 c2.b.data_ptr(), 1 | nat.WEIGHTS_X6 | (nat.ACT_EXP if x6 == "act_exp" else 0),
                 c3.w.data_ptr(), c3.b.data_ptr(), y_len, out.data_ptr(),
                 d.data_ptr(), wsb, stream())
        torch.cuda.synchronize()
        assert not torch.isnan(out).any()
        close(out, fp32, rel=5e-5)
    torch.cuda.synchronize()
    if L <= 2000:
        x64 = x.double()
        hid = F.elu(causal_conv1d(F.elu(x64), w1.double(), b1.double()))
        blk = F.elu(x64 + causal_conv1d(hid, w2.double(), b2.double()))
        want = causal_conv1d(blk, w3.double(), b3.double())[..., :y_len]
        close(out.cpu().view(B, 1, y_len), want, rel=5e-5)
    else:  # long inputs: against the two separate kernels
        h = torch.empty_like(xd)
        nat.call("fm_resblock", xd.data_ptr(), B, L, 64, c1.w.data_ptr(), c1.b.data_ptr(),
                 c2.w.data_ptr(), c2.b.data_ptr(), 1, h.data_ptr(), stream())
        ws = torch.empty(WS_BYTES // 4, device=DEV)
        ref = torch.empty(B, y_len, 1, device=DEV)
        nat.call("fm_conv1d", h.data_ptr(), B, L, 64, c3.w.data_ptr(), c3.b.data_ptr(), 1, 3, 1, 0, 0,
                 None, ref.data_ptr(), y_len, ws.data_ptr(), WS_BYTES, stream())
        torch.cuda.synchronize()
        err = (out.cpu() - ref.cpu().view(B, y_len)).abs().max().item()
        assert err <= 1e-5 * max(1.0, ref.abs().max().item()), err


def test_conv1d_crop(ws):
    g = torch.Generator().manual_seed(5)
    x = torch.randn(2, 8, 100, generator=g)
    w = torch.randn(1, 8, 3, generator=g)
    b = torch.randn(1, generator=g)
    got = run_conv(x, w, b, 1, "constant", 0, ws, y_len=93)
    want = causal_conv1d(x.double(), w.double(), b.double())[..., :93]
    close(got, want)


@pytest.mark.parametrize("B,cin,cout,stride,L", [
    (1, 1024, 512, 8, 250), (2, 512, 256, 6, 40), (1, 256, 128, 5, 300),
    (1, 128, 64, 4, 1000), (1, 4, 2, 2, 7), (2, 8, 4, 2, 1), (1, 128, 64, 4, 40000),
    (1, 128, 64, 4, 60000)])
@pytest.mark.parametrize("x6", [False, True], ids=["fp32", "bf16x6"])
def test_conv_transpose1d(B, cin, cout, stride, L, x6, ws):
    g = torch.Generator().manual_seed(cin + L)
    x = torch.randn(B, cin, L, generator=g)
    w = torch.randn(cin, cout, 2 * stride, generator=g) / math.sqrt(cin)
    b = torch.randn(cout, generator=g) * 0.1
    layer = _ConvT(w.to(DEV), b.to(DEV), stride)
    flags = 0
    if x6:
        layer.w, flags = with_planes(layer.w), nat.WEIGHTS_X6
    xd = x.transpose(1, 2).contiguous().to(DEV)
    y = torch.empty((B, L * stride, cout), device=DEV)
    nat.call("fm_conv_transpose1d", xd.data_ptr(), B, L, cin, layer.w.data_ptr(), layer.b.data_ptr(),
             cout, 2 * stride, stride, flags, None, y.data_ptr(), ws.data_ptr(), WS_BYTES, stream())
    torch.cuda.synchronize()
    want = causal_conv_transpose1d(x.double(), w.double(), b.double(), stride)
    close(y.cpu().transpose(1, 2), want)
    close_dot(y.cpu().transpose(1, 2), want,
              causal_conv_transpose1d(x.double().abs(), w.double().abs(), b.double().abs(), stride))


def run_linear(x, w, flags=0, res=None, scale=None, ws=None, out=None):
    """y = x @ w^T with w given as [out, in] (the packed W^T layout)."""
    rows, k = x.shape
    n = w.shape[0]
    y = torch.empty((rows, n), device=DEV) if out is None else out
    nat.call("fm_linear", x.data_ptr(), rows, k, w.data_ptr(), n, flags,
             None if res is None else res.data_ptr(), None if scale is None else scale.data_ptr(),
             y.data_ptr(), ws.data_ptr(), WS_BYTES, stream())
    torch.cuda.synchronize()
    return y


@pytest.mark.parametrize("rows,k,n", [(250, 512, 1536), (4000, 512, 2048), (250, 2048, 512),
                                      (1, 512, 512), (37, 16, 48), (125, 512, 512),
                                      (60000, 256, 256), (60001, 96, 200),
                                      (4000, 512, 1536), (4001, 512, 1536),  # 192x128 tiles
                                      (2500, 512, 512), (4001, 512, 512),    # 64x128 tiles
                                      (2500, 512, 2048)])
@pytest.mark.parametrize("x6", [False, True], ids=["fp32", "bf16x6"])
def test_linear_epilogues(rows, k, n, x6, ws):
    g = torch.Generator().manual_seed(rows + k + n)
    x = torch.randn(rows, k, generator=g)
    w = torch.randn(n, k, generator=g) * 0.05
    xd, wd = x.to(DEV), w.to(DEV)
    f = 0
    if x6:
        wd, f = with_planes(wd), nat.WEIGHTS_X6
    close(run_linear(xd, wd, f, ws=ws).cpu(), x.double() @ w.double().t())
    close_dot(run_linear(xd, wd, f, ws=ws).cpu(), x.double() @ w.double().t(),
              x.double().abs() @ w.double().abs().t())
    close(run_linear(xd, wd, nat.EPI_GELU | f, ws=ws).cpu(), F.gelu(x.double() @ w.double().t()))
    res = torch.randn(rows, n, generator=g)
    scale = torch.rand(n, generator=g) * 0.1
    h = res.to(DEV)
    run_linear(xd, wd, nat.EPI_RES_SCALE | f, res=h, scale=scale.to(DEV), ws=ws, out=h)  # in place
    close(h.cpu(), res.double() + scale.double() * (x.double() @ w.double().t()))


@pytest.mark.parametrize("rows,c", [(250, 512), (1, 512), (33, 16), (4000, 512)])
def test_layer_norm(rows, c):
    g = torch.Generator().manual_seed(rows)
    x = torch.randn(rows, c, generator=g) * 3 + 1
    w = torch.rand(c, generator=g) + 0.5
    b = torch.randn(c, generator=g)
    xd, y = x.to(DEV), torch.empty(rows, c, device=DEV)
    wd, bd = w.to(DEV), b.to(DEV)  # keep device copies alive across the call
    nat.call("fm_layer_norm", xd.data_ptr(), wd.data_ptr(), bd.data_ptr(), rows, c,
             1e-5, y.data_ptr(), stream())
    torch.cuda.synchronize()
    close(y.cpu(), F.layer_norm(x.double(), (c,), w.double(), b.double(), 1e-5))


def attention_reference(qkv, B, T, H, D, window, cos, sin):
    """float64 RoPE + causal window softmax attention, the oracle's formulas."""
    q, k, v = qkv.double().view(B, T, 3, H, D).unbind(2)
    q, k, v = (t.transpose(1, 2) for t in (q, k, v))
    c, s = cos.double()[None, None], sin.double()[None, None]
    rot = MimiOracle._rotate_half
    q = q * c + rot(q) * s
    k = k * c + rot(k) * s
    i = torch.arange(T)
    allowed = (i[None, :] <= i[:, None]) & (i[None, :] > i[:, None] - window)
    scores = (q @ k.transpose(-1, -2)) / math.sqrt(D)
    scores = scores.masked_fill(~allowed, float("-inf"))
    o = torch.softmax(scores, -1) @ v
    return o.transpose(1, 2).reshape(B * T, H * D)


@pytest.mark.parametrize("B,T,H,D,window", [(1, 250, 8, 64, 250), (1, 251, 8, 64, 250),
                                            (2, 700, 8, 64, 250), (1, 1, 8, 64, 250),
                                            (16, 125, 8, 64, 250), (8, 300, 8, 64, 250), (2, 18, 2, 8, 8),
                                            # whole-sequence kernel (>= 128 sequence-heads, T <= 256)
                                            (16, 250, 8, 64, 250), (16, 256, 8, 64, 250),
                                            (20, 200, 8, 64, 64), (32, 97, 8, 64, 250), (128, 1, 8, 64, 250),
                                            # 64-query chunked kernel (>= 512 queries, < 128 sequence-heads)
                                            (1, 2500, 8, 64, 250), (1, 1000, 8, 64, 64), (3, 513, 8, 64, 250)])
def test_window_attention(B, T, H, D, window):
    g = torch.Generator().manual_seed(T + H)
    qkv = torch.randn(B * T, 3 * H * D, generator=g)
    cfg = MimiConfig(head_dim=D, hidden_size=H * D, num_attention_heads=H, num_key_value_heads=H)
    cos, sin = rope_tables(cfg, T)
    out = torch.empty(B * T, H * D, device=DEV)
    qkv_d, cos_d, sin_d = qkv.to(DEV), cos.to(DEV), sin.to(DEV)
    nat.call("fm_window_attention", qkv_d.data_ptr(), 3 * H * D, 0, H * D, 2 * H * D,
             cos_d.data_ptr(), sin_d.data_ptr(), B, T, H, H, D, window,
             1.0 / math.sqrt(D), out.data_ptr(), H * D, stream())
    torch.cuda.synchronize()
    close(out.cpu(), attention_reference(qkv, B, T, H, D, window, cos, sin), rel=5e-5)


@pytest.mark.parametrize("B,T", [(1, 300), (16, 250), (1, 700)])
def test_window_attention_grouped_kv_heads(B, T):
    """kv_heads < heads: head h reads K/V head h // (heads / kv_heads), for the
    16-query, whole-sequence and long-sequence kernels."""
    H, KV, D, window = 8, 2, 64, 250
    g = torch.Generator().manual_seed(B * 7 + T)
    ld = (H + 2 * KV) * D
    qkv = torch.randn(B * T, ld, generator=g)
    cfg = MimiConfig()
    cos, sin = rope_tables(cfg, T)
    # Expanded to one K/V per query head, the reference formulas apply unchanged.
    q = qkv[:, :H * D].view(B * T, H, D)
    k = qkv[:, H * D:(H + KV) * D].view(B * T, KV, D).repeat_interleave(H // KV, dim=1)
    v = qkv[:, (H + KV) * D:].view(B * T, KV, D).repeat_interleave(H // KV, dim=1)
    full = torch.cat([q, k, v], 1).reshape(B * T, 3 * H * D)
    out = torch.empty(B * T, H * D, device=DEV)
    qkv_d, cos_d, sin_d = qkv.to(DEV), cos.to(DEV), sin.to(DEV)
    nat.call("fm_window_attention", qkv_d.data_ptr(), ld, 0, H * D, (H + KV) * D, cos_d.data_ptr(),
             sin_d.data_ptr(), B, T, H, KV, D, window, 1.0 / math.sqrt(D), out.data_ptr(), H * D,
             stream())
    torch.cuda.synchronize()
    close(out.cpu(), attention_reference(full, B, T, H, D, window, cos, sin), rel=5e-5)


@pytest.mark.parametrize("B,T", [(1, 300), (16, 250)])
def test_window_attention_prerotated(B, T):
    """NULL RoPE tables: q/k are consumed as given (rotated by their producer)."""
    H, D, window = 8, 64, 250
    g = torch.Generator().manual_seed(5)
    qkv = torch.randn(B * T, 3 * H * D, generator=g)
    cfg = MimiConfig()
    cos, sin = rope_tables(cfg, T)
    q, k, v = qkv.view(B, T, 3, H, D).unbind(2)
    rot = MimiOracle._rotate_half
    c, s_ = cos[None, :, None], sin[None, :, None]
    pre = torch.stack([q * c + rot(q) * s_, k * c + rot(k) * s_, v], 2).reshape(B * T, 3 * H * D)
    out = torch.empty(B * T, H * D, device=DEV)
    pre_d = pre.contiguous().to(DEV)
    nat.call("fm_window_attention", pre_d.data_ptr(), 3 * H * D, 0, H * D, 2 * H * D, None, None,
             B, T, H, H, D, window, 1.0 / math.sqrt(D), out.data_ptr(), H * D, stream())
    torch.cuda.synchronize()
    close(out.cpu(), attention_reference(qkv, B, T, H, D, window, cos, sin), rel=5e-5)


PACKED = {"packed": True, "x6": False}


def run_row_linear(x, w, flags=0, ln=None, rope=None, res=None, scale=None, out=None):
    rows, k = x.shape
    n = w.shape[0]
    y = torch.empty(rows, n, device=DEV) if out is None else out
    g, b = ln if ln is not None else (None, None)
    cos, sin, rope_cols, per_seq = rope if rope is not None else (None, None, 0, 1)
    p = lambda t: None if t is None else t.data_ptr()  # noqa: E731
    name, wp = "fm_row_linear", w
    if PACKED["x6"]:
        wp, flags = with_planes(w), flags | nat.WEIGHTS_X6
    elif PACKED["packed"]:
        wp = torch.empty_like(w)
        nat.call("fm_pack_row_weights", w.data_ptr(), n, k, wp.data_ptr(), stream())
        name = "fm_row_linear_packed"
    nat.call(name, x.data_ptr(), rows, k, p(g), p(b), 1e-5, wp.data_ptr(), n, flags,
             p(res), p(scale), p(cos), p(sin), rope_cols, per_seq, y.data_ptr(), stream())
    torch.cuda.synchronize()
    return y


@pytest.fixture(params=["rowmajor", "packed", "bf16x6"])
def weight_layout(request):
    PACKED["packed"] = request.param == "packed"
    PACKED["x6"] = request.param == "bf16x6"
    yield request.param
    PACKED["packed"] = False
    PACKED["x6"] = False


def test_pack_row_weights_layout():
    n, k = 48, 128
    w = torch.arange(n * k, dtype=torch.float32).view(n, k)
    wd = w.to(DEV)
    out = torch.empty_like(wd)
    nat.call("fm_pack_row_weights", wd.data_ptr(), n, k, out.data_ptr(), stream())
    torch.cuda.synchronize()
    got = out.cpu().view(-1, 4)
    for i in (0, 1, 63, 64, 255, 256, 777, got.shape[0] - 1):
        lane, q = i % 64, i // 64
        t, q2 = q % 4, q // 4
        kp, nt = q2 % (k // 64), q2 // (k // 64)
        row, col = 16 * nt + lane % 16, 64 * kp + 16 * (lane // 16) + 4 * t
        assert torch.equal(got[i], w[row, col:col + 4]), i


@pytest.mark.parametrize("rows", [250, 1, 33, 500, 4000])
def test_row_linear(rows, weight_layout):
    """LayerNorm prologue + RoPE / GELU / LayerScale-residual epilogues vs float64."""
    g = torch.Generator().manual_seed(rows)
    k, H, D = 512, 8, 64
    x = torch.randn(rows, k, generator=g) * 2 + 0.5
    gamma, beta = torch.rand(k, generator=g) + 0.5, torch.randn(k, generator=g) * 0.1
    wqkv = torch.randn(3 * k, k, generator=g) * 0.04
    w1 = torch.randn(2048, k, generator=g) * 0.04
    wo = torch.randn(k, k, generator=g) * 0.04
    T = 250 if rows >= 250 else rows
    cos, sin = rope_tables(MimiConfig(), T)
    d = {name: t.to(DEV) for name, t in dict(x=x, gamma=gamma, beta=beta, wqkv=wqkv, w1=w1, wo=wo,
                                             cos=cos, sin=sin).items()}
    xn = F.layer_norm(x.double(), (k,), gamma.double(), beta.double(), 1e-5)
    # Plain product and LN + product.
    close(run_row_linear(d["x"], d["wo"]).cpu(), x.double() @ wo.double().t())
    close_dot(run_row_linear(d["x"], d["wo"]).cpu(), x.double() @ wo.double().t(),
              x.double().abs() @ wo.double().abs().t())
    # LN + qkv + RoPE on q and k (positions row % T).
    got = run_row_linear(d["x"], d["wqkv"], ln=(d["gamma"], d["beta"]),
                         rope=(d["cos"], d["sin"], 2 * k, T)).cpu()
    want = xn @ wqkv.double().t()
    t = torch.arange(rows) % T
    c, s = cos.double()[t][:, None], sin.double()[t][:, None]
    qk = want[:, : 2 * k].reshape(rows, 2 * H, D)
    want[:, : 2 * k] = (qk * c + MimiOracle._rotate_half(qk) * s).reshape(rows, 2 * k)
    close(got, want)
    # LN + fc1 + GELU.
    close(run_row_linear(d["x"], d["w1"], nat.EPI_GELU, ln=(d["gamma"], d["beta"])).cpu(),
          F.gelu(xn @ w1.double().t()))
    # LayerScale residual, in place.
    res = torch.randn(rows, k, generator=g)
    scale = torch.rand(k, generator=g) * 0.1
    h = res.to(DEV)
    run_row_linear(d["x"], d["wo"], nat.EPI_RES_SCALE, res=h, scale=scale.to(DEV), out=h)
    close(h.cpu(), res.double() + scale.double() * (x.double() @ wo.double().t()))


@pytest.mark.parametrize("rows", [250, 1, 17, 1000])
def test_row_linear_long_k(rows, weight_layout):
    """K = 2048 streamed path (fc2): plain, GELU and in-place LayerScale residual."""
    g = torch.Generator().manual_seed(rows + 7)
    x = torch.randn(rows, 2048, generator=g)
    w = torch.randn(512, 2048, generator=g) * 0.02
    xd, wd = x.to(DEV), w.to(DEV)
    want = x.double() @ w.double().t()
    close(run_row_linear(xd, wd).cpu(), want)
    close_dot(run_row_linear(xd, wd).cpu(), want, x.double().abs() @ w.double().abs().t())
    close(run_row_linear(xd, wd, nat.EPI_GELU).cpu(), F.gelu(want))
    res = torch.randn(rows, 512, generator=g)
    scale = torch.rand(512, generator=g) * 0.1
    h = res.to(DEV)
    run_row_linear(xd, wd, nat.EPI_RES_SCALE, res=h, scale=scale.to(DEV), out=h)
    close(h.cpu(), res.double() + scale.double() * want)


def test_row_linear_rejects():
    lib = nat.library()
    assert lib.fm_row_linear_supported(512, 1536) and lib.fm_row_linear_supported(2048, 512)
    assert not lib.fm_row_linear_supported(1024, 512) and not lib.fm_row_linear_supported(512, 100)
    x = torch.zeros(4, 1024, device=DEV)
    w = torch.zeros(512, 1024, device=DEV)
    with pytest.raises(nat.NativeError, match="unsupported"):
        run_row_linear(x, w)
    x2, w2, gb = torch.zeros(4, 2048, device=DEV), torch.zeros(512, 2048, device=DEV), torch.ones(2048, device=DEV)
    with pytest.raises(nat.NativeError, match="unsupported"):
        run_row_linear(x2, w2, ln=(gb, gb))


@pytest.mark.parametrize("B,L,ci,co,k,s,flags", [
    (1, 13, 1, 64, 7, 1, 0), (2, 40, 64, 32, 3, 1, nat.ELU_IN | nat.EPI_ELU),
    (1, 22, 128, 256, 10, 5, 0), (3, 9, 512, 512, 4, 2, 0), (1, 18, 32, 64, 1, 1, 0)])
def test_conv1d_valid(B, L, ci, co, k, s, flags, ws):
    """No-padding conv (streaming): output t reads rows t*s .. t*s + k - 1."""
    g = torch.Generator().manual_seed(L * k + ci)
    x = torch.randn(B, ci, L, generator=g)
    w = torch.randn(co, ci, k, generator=g) * 0.1
    b = torch.randn(co, generator=g)
    layer = _Conv(w.to(DEV), b.to(DEV), s)
    xd = x.transpose(1, 2).contiguous().to(DEV)
    rows = (L - k) // s + 1
    y = torch.empty(B, rows, co, device=DEV)
    nat.call("fm_conv1d_valid", xd.data_ptr(), B, L, ci, layer.w.data_ptr(), layer.b.data_ptr(),
             co, k, s, flags, None, y.data_ptr(), ws.data_ptr(), WS_BYTES, stream())
    torch.cuda.synchronize()
    xin = F.elu(x.double()) if flags & nat.ELU_IN else x.double()
    want = F.conv1d(xin, w.double(), b.double(), s)
    if flags & nat.EPI_ELU:
        want = F.elu(want)
    close(y.cpu().transpose(1, 2), want)
    with pytest.raises(nat.NativeError, match="bad argument"):
        nat.call("fm_conv1d_valid", xd.data_ptr(), B, k - 1, ci, layer.w.data_ptr(), None, co, k, s,
                 0, None, y.data_ptr(), ws.data_ptr(), WS_BYTES, stream())


@pytest.mark.parametrize("B,T,q_start,window", [(1, 260, 249, 250), (2, 300, 249, 250),
                                                (1, 10, 9, 250), (3, 12, 4, 8), (1, 64, 0, 250),
                                                (1, 1100, 300, 250), (2, 700, 150, 100)])
def test_window_attention_rows_with_cached_keys(B, T, q_start, window):
    """Queries at rows q_start.. over all rows as keys (a KV cache in front)."""
    H, D = 8, 64
    g = torch.Generator().manual_seed(T + q_start)
    qkv = torch.randn(B * T, 3 * H * D, generator=g)
    out = torch.empty(B * (T - q_start), H * D, device=DEV)
    qd = qkv.to(DEV)
    nat.call("fm_window_attention_rows", qd.data_ptr(), 3 * H * D, 0, H * D, 2 * H * D, None, None,
             B, T, q_start, H, H, D, window, 1.0 / math.sqrt(D), out.data_ptr(), H * D, stream())
    torch.cuda.synchronize()
    zeros = torch.zeros(T, D)
    cos1 = torch.ones(T, D)  # identity rotation: q, k taken as given
    want = attention_reference(qkv, B, T, H, D, window, cos1, zeros)
    want = want.view(B, T, H * D)[:, q_start:].reshape(-1, H * D)
    close(out.cpu(), want, rel=5e-5)


@pytest.mark.parametrize("rows,T,H,D", [(250, 250, 8, 64), (7, 7, 2, 8), (40, 20, 2, 16)])
def test_apply_rope_in_place(rows, T, H, D):
    g = torch.Generator().manual_seed(rows + D)
    x = torch.randn(rows, 3 * H * D, generator=g)
    cfg = MimiConfig(head_dim=D, hidden_size=H * D, num_attention_heads=H, num_key_value_heads=H)
    cos, sin = rope_tables(cfg, T)
    xd, cd, sd = x.to(DEV), cos.to(DEV), sin.to(DEV)
    nat.call("fm_apply_rope", xd.data_ptr(), rows, 3 * H * D, 2 * H * D, D, cd.data_ptr(),
             sd.data_ptr(), T, stream())
    torch.cuda.synchronize()
    t = torch.arange(rows) % T
    qk = x[:, : 2 * H * D].reshape(rows, 2 * H, D)
    c, s_ = cos[t][:, None], sin[t][:, None]
    want = x.clone()
    want[:, : 2 * H * D] = (qk * c + MimiOracle._rotate_half(qk) * s_).reshape(rows, -1)
    assert torch.equal(xd.cpu(), want)  # same rounding steps as the reference's _apply_rope


def test_elu_accuracy_dense(ws):
    """ELU through an identity 1x1 conv (EPI_ELU) against float64 expm1 over
    a dense grid of x <= 0, plus x > 0 passthrough: within 4 ulp."""
    x = torch.cat([-torch.logspace(-8, 2, 200_000, dtype=torch.float64),
                   torch.linspace(-1, 0, 100_001, dtype=torch.float64),
                   torch.logspace(-8, 2, 1000, dtype=torch.float64)]).float()
    n = x.numel() // 4 * 4
    x = x[:n]
    w = torch.eye(4).view(4, 4, 1)
    y = run_conv(x.view(1, n // 4, 4).transpose(1, 2), w, None, 1, 0, nat.EPI_ELU, ws)
    got = y.transpose(1, 2).reshape(-1).double()
    want = torch.where(x > 0, x.double(), torch.expm1(x.double()))
    ulp = torch.nextafter(want.float().abs(), torch.tensor(float("inf"))).double() - want.abs().float().double()
    err = ((got - want).abs() / ulp.clamp(min=1e-45)).max().item()
    assert err <= 4.0, f"max error {err:.2f} ulp"


def prepare_codebooks(embed_sum, usage):
    n, e, d = embed_sum.shape
    emb = torch.empty(n, e, d, device=DEV)
    emb_t = torch.empty(n, d, e, device=DEV)
    norms = torch.empty(n, e, device=DEV)
    es_d, us_d = embed_sum.to(DEV).contiguous(), usage.to(DEV).contiguous()
    for j in range(n):
        nat.call("fm_rvq_prepare_codebook", es_d[j].data_ptr(),
                 us_d[j].data_ptr(), e, d, 1e-5, emb[j].data_ptr(),
                 emb_t[j].data_ptr(), norms[j].data_ptr(), stream())
    return emb, emb_t, norms


def rvq_encode_gpu(x, emb, emb_t, norms, T, nq):
    M, d = x.shape
    e = emb.shape[1]
    B = M // T
    codes = torch.empty(B, nq, T, dtype=torch.int64, device=DEV)
    wsb = nat.library().fm_rvq_workspace_bytes(M, d, e)
    ws = torch.empty((wsb + 3) // 4, device=DEV)
    xd = x.to(DEV).contiguous()
    nat.call("fm_rvq_encode", xd.data_ptr(), d, M, T, d, e, nq, emb.data_ptr(), emb_t.data_ptr(),
             norms.data_ptr(), codes.data_ptr(), nq * T, ws.data_ptr(), wsb, stream())
    torch.cuda.synchronize()
    return codes.cpu()


def rvq_encode_oracle(x, embeds, T):
    """The reference's residual loop (model.py:2408-2428) on flat rows."""
    residual = x.clone()
    out = []
    for e in embeds:
        idx = MimiOracle.nearest(residual, e)
        out.append(idx)
        residual = residual - F.embedding(idx, e)
    codes = torch.stack(out)  # [nq, M]
    nq, M = codes.shape
    return codes.view(nq, M // T, T).transpose(0, 1)


@pytest.mark.parametrize("B,T,nq,e,d", [
    (1, 125, 8, 2048, 256),    # 32-entry chunks, 4 k-parts
    (4, 63, 7, 2048, 256),
    (8, 100, 4, 2048, 256),    # 64-entry chunks, 2 k-parts
    (64, 125, 32, 2048, 256),  # 512-entry chunks, 1 k-part
    (1, 1, 3, 2048, 256),
    (3, 100, 3, 1000, 128),    # ragged last chunk
    (2, 70, 3, 100, 64),
    (2, 40, 3, 48, 8),         # general kernel (dim not in {64, 128, 256})
    # 64-row blocks (>= 1024 rows): two query tiles per codebook fragment
    (16, 125, 8, 2048, 256),
    (11, 100, 5, 1000, 128),   # ragged last chunk
    (17, 61, 3, 2048, 64),     # partial last row block
])
def test_rvq_encode_matches_reference_loop(B, T, nq, e, d):
    g = torch.Generator().manual_seed(B * T + nq + e + d)
    embed_sum = torch.randn(nq, e, d, generator=g) / 16
    usage = torch.ones(nq, e)
    x = torch.randn(B * T, d, generator=g) * 0.3
    emb, emb_t, norms = prepare_codebooks(embed_sum, usage)
    got = rvq_encode_gpu(x, emb, emb_t, norms, T, nq)
    embeds = [embed_sum[j] / usage[j].clamp(min=1e-5)[:, None] for j in range(nq)]
    want = rvq_encode_oracle(x, embeds, T)
    flat = want.transpose(0, 1).reshape(nq, B * T)

    def rerun(rows, j0, count):
        return rvq_encode_gpu(rows, emb[j0:], emb_t[j0:], norms[j0:], 1, count)[:, :, 0].t()

    # Near-ties within FP32 summation-order noise are certified (and the rest
    # of each such chain re-run from the reference's residual); report them.
    report = check_codes(got, want, reference_rvq_rows(x, embeds, flat), embeds, nq, rerun,
                         allow=(max(2, B * T * nq // 2000), 1e-6))
    print(f"rvq B={B} T={T} nq={nq}: {report.summary()}")


def test_rvq_non_finite_rows_give_reference_codes():
    """NaN / Inf residual rows: torch's argmin returns the first NaN distance
    (index 0 for an all-NaN row); the kernel must give the same in-range codes."""
    B, T, nq, e, d = 1, 96, 3, 2048, 256
    g = torch.Generator().manual_seed(17)
    embed_sum = torch.randn(nq, e, d, generator=g) / 16
    x = torch.randn(B * T, d, generator=g) * 0.3
    x[3, 5] = float("nan")
    x[40] = float("nan")
    x[41, 0] = float("inf")
    x[77, 9] = float("-inf")
    emb, emb_t, norms = prepare_codebooks(embed_sum, torch.ones(nq, e))
    got = rvq_encode_gpu(x, emb, emb_t, norms, T, nq)
    want = rvq_encode_oracle(x, [embed_sum[j] for j in range(nq)], T)
    assert ((got >= 0) & (got < e)).all()
    assert torch.equal(got, want)


@pytest.mark.parametrize("B,T,nsem,nac,e,d", [
    (1, 125, 1, 7, 2048, 256),    # 32-entry chunks, 4 k-parts
    (16, 125, 1, 7, 2048, 256),   # 128-entry chunks
    (64, 125, 1, 31, 2048, 256),  # long acoustic chain
    (3, 100, 2, 3, 1000, 128),    # ragged last chunk, two semantic codebooks
    (2, 70, 1, 2, 100, 64),
    (1, 33, 1, 0, 2048, 256),     # semantic only
    (1, 33, 0, 3, 2048, 256),     # acoustic only
    (2, 40, 1, 2, 48, 8),         # general kernel: branches one after the other
    # <= 128 rows at dim 256: the persistent one-launch chain (must equal the
    # per-step launches bit for bit)
    (1, 128, 1, 7, 2048, 256),    # four full 32-row tiles
    (1, 1, 1, 7, 2048, 256),      # one row
    (1, 97, 2, 5, 1000, 256),     # ragged entries (blocks past the codebook), partial tile
    (2, 33, 1, 31, 2048, 256),    # long acoustic chain, rows across two batch items
    (1, 64, 3, 1, 2048, 256),     # longer semantic chain than acoustic
])
def test_rvq_encode_split_matches_two_branches(B, T, nsem, nac, e, d):
    """Shared-launch split encode == the two branches encoded separately (bit-exact codes)."""
    g = torch.Generator().manual_seed(B * T + nsem + nac + e + d)
    n = nsem + nac
    embed_sum = torch.randn(n, e, d, generator=g) / 16
    emb, emb_t, norms = prepare_codebooks(embed_sum, torch.ones(n, e))
    M = B * T
    x = (torch.randn(M, 2 * d, generator=g) * 0.3).to(DEV)
    lib = nat.library()
    codes = torch.full((B, n, T), -1, dtype=torch.int64, device=DEV)
    wsb = lib.fm_rvq_split_workspace_bytes(M, d, e)
    ws = torch.empty((wsb + 3) // 4, device=DEV)
    nat.call("fm_rvq_encode_split", x.data_ptr(), 2 * d, M, T, d, e, nsem, nac, emb.data_ptr(),
             emb_t.data_ptr(), norms.data_ptr(), codes.data_ptr(), n * T, ws.data_ptr(), wsb, stream())
    want = torch.full((B, n, T), -2, dtype=torch.int64, device=DEV)
    wsb1 = lib.fm_rvq_workspace_bytes(M, d, e)
    ws1 = torch.empty((wsb1 + 3) // 4, device=DEV)
    for col, first, count in ((0, 0, nsem), (d, nsem, nac)):
        if count == 0:
            continue
        nat.call("fm_rvq_encode", x.data_ptr() + col * 4, 2 * d, M, T, d, e, count,
                 emb[first].data_ptr(), emb_t[first].data_ptr(), norms[first].data_ptr(),
                 want.data_ptr() + first * T * 8, n * T, ws1.data_ptr(), wsb1, stream())
    torch.cuda.synchronize()
    assert torch.equal(codes.cpu(), want.cpu())
    # Empty input is a no-op.
    nat.call("fm_rvq_encode_split", x.data_ptr(), 2 * d, 0, T, d, e, nsem, nac, emb.data_ptr(),
             emb_t.data_ptr(), norms.data_ptr(), codes.data_ptr(), n * T, ws.data_ptr(), wsb, stream())


@pytest.mark.parametrize("B,T,nsem,nac,e,spin", [
    (1, 128, 1, 7, 2048, "0"),    # every wait gives up at the first resolve
    (1, 97, 2, 5, 1000, "0"),     # ragged entries and a partial tile
    (2, 33, 1, 31, 2048, "0"),    # long acoustic chain
    (1, 125, 1, 7, 2048, "3"),    # a few polls: waits give up at different steps
])
def test_rvq_chain_recomputes_alone_when_a_wait_gives_up(B, T, nsem, nac, e, spin, monkeypatch):
    """When a wait of the one-launch chain for other blocks' partials gives
    up, block 0 of the group computes the whole chain again alone, from all
    entries' distances with the same arithmetic: the codes still equal the
    per-branch launches bit for bit.  The wait limit is lowered from the
    host (FM_RVQ_CHAIN_SPIN), so every kernel still ends normally."""
    monkeypatch.setenv("FM_RVQ_CHAIN_SPIN", spin)
    d = 256
    g = torch.Generator().manual_seed(B * T + nsem + nac + e)
    n = nsem + nac
    emb, emb_t, norms = prepare_codebooks(torch.randn(n, e, d, generator=g) / 16, torch.ones(n, e))
    M = B * T
    x = (torch.randn(M, 2 * d, generator=g) * 0.3).to(DEV)
    lib = nat.library()
    codes = torch.full((B, n, T), -1, dtype=torch.int64, device=DEV)
    wsb = lib.fm_rvq_split_workspace_bytes(M, d, e)
    ws = torch.empty((wsb + 3) // 4, device=DEV)
    nat.call("fm_rvq_encode_split", x.data_ptr(), 2 * d, M, T, d, e, nsem, nac, emb.data_ptr(),
             emb_t.data_ptr(), norms.data_ptr(), codes.data_ptr(), n * T, ws.data_ptr(), wsb, stream())
    want = torch.full((B, n, T), -2, dtype=torch.int64, device=DEV)
    wsb1 = lib.fm_rvq_workspace_bytes(M, d, e)
    ws1 = torch.empty((wsb1 + 3) // 4, device=DEV)
    for col, first, count in ((0, 0, nsem), (d, nsem, nac)):
        nat.call("fm_rvq_encode", x.data_ptr() + col * 4, 2 * d, M, T, d, e, count,
                 emb[first].data_ptr(), emb_t[first].data_ptr(), norms[first].data_ptr(),
                 want.data_ptr() + first * T * 8, n * T, ws1.data_ptr(), wsb1, stream())
    torch.cuda.synchronize()
    assert torch.equal(codes.cpu(), want.cpu())


def test_rvq_tie_picks_lowest_index():
    e, d = 256, 256
    g = torch.Generator().manual_seed(9)
    base = torch.randn(e, d, generator=g) / 16
    base[200] = base[17]  # exact duplicate entries: distance ties
    base[255] = base[17]
    x = base[17:18].repeat(64, 1) + 1e-3 * torch.randn(64, d, generator=g)
    emb, emb_t, norms = prepare_codebooks(base[None], torch.ones(1, e))
    got = rvq_encode_gpu(x, emb, emb_t, norms, 64, 1)
    want = rvq_encode_oracle(x, [base], 64)
    assert torch.equal(got, want)
    assert (got == 17).all()


def test_rvq_prepare_divides_by_clamped_usage():
    g = torch.Generator().manual_seed(4)
    es = torch.randn(1, 64, 32, generator=g)
    usage = torch.rand(1, 64, generator=g) + 0.5
    usage[0, 3] = 0.0  # clamps to 1e-5
    emb, emb_t, _ = prepare_codebooks(es, usage)
    want = es[0] / usage[0].clamp(min=1e-5)[:, None]
    assert torch.equal(emb[0].cpu(), want)
    assert torch.equal(emb_t[0].cpu(), want.t())


@pytest.mark.parametrize("B,nq,T,nsem", [(1, 8, 125, 1), (2, 32, 13, 1), (3, 1, 5, 1), (1, 4, 3, 1)])
def test_rvq_decode_gather_sum_is_exact(B, nq, T, nsem):
    g = torch.Generator().manual_seed(nq * T)
    e, d = 2048, 256
    embeds = torch.randn(nq, e, d, generator=g) / 16
    codes = torch.randint(0, e, (B, nq, T), generator=g)
    out = torch.empty(B * T, 2 * d, device=DEV)
    codes_d, embeds_d = codes.to(DEV), embeds.to(DEV)
    nat.call("fm_rvq_decode", codes_d.data_ptr(), B, nq, T, nsem, embeds_d.data_ptr(),
             e, d, out.data_ptr(), stream())
    torch.cuda.synchronize()
    # Reference order (model.py:2439-2441): float32 zero, then codebooks left to right.
    sem = torch.zeros(())
    for j in range(nsem):
        sem = sem + F.embedding(codes[:, j], embeds[j])
    ac = torch.zeros(())
    for j in range(nsem, nq):
        ac = ac + F.embedding(codes[:, j], embeds[j])
    got = out.cpu().view(B, T, 2 * d)
    assert torch.equal(got[..., :d], sem.expand(B, T, d))
    assert torch.equal(got[..., d:], ac.expand(B, T, d))


@pytest.mark.parametrize("B,T", [(1, 125), (2, 63), (3, 1), (1, 31)])
def test_row_linear_packed_upsample_matches_two_launches(B, T):
    """Output projection + depthwise k4 s2 upsample in one launch gives the
    bits of fm_row_linear_packed followed by fm_upsample_depthwise, sequence
    starts included (frames whose 16-row block begins inside another sequence)."""
    g = torch.Generator().manual_seed(B * 100 + T)
    N, K = 512, 512
    x = torch.randn(B * T, K, generator=g).to(DEV)
    w = (torch.randn(N, K, generator=g) * 0.05).to(DEV)
    up = (torch.randn(N, 1, 4, generator=g) * 0.5).to(DEV)
    wp = torch.empty_like(w)
    nat.call("fm_pack_row_weights", w.data_ptr(), N, K, wp.data_ptr(), stream())
    h = torch.empty(B * T, N, device=DEV)
    nat.call("fm_row_linear_packed", x.data_ptr(), B * T, K, None, None, 1e-5, wp.data_ptr(), N, 0,
             None, None, None, None, 0, T, h.data_ptr(), stream())
    want = torch.empty(B, 2 * T, N, device=DEV)
    nat.call("fm_upsample_depthwise", h.data_ptr(), B, T, N, up.data_ptr(), 4, 2, want.data_ptr(), stream())
    got = torch.full((B, 2 * T, N), float("nan"), device=DEV)
    nat.call("fm_row_linear_packed_upsample", x.data_ptr(), B * T, K, wp.data_ptr(), N, T, up.data_ptr(),
             got.data_ptr(), stream())
    torch.cuda.synchronize()
    assert torch.equal(got, want)
    ref = F.conv_transpose1d((x.double().cpu() @ w.double().cpu().t()).view(B, T, N).transpose(1, 2),
                             up.double().cpu(), None, 2, 0, 0, N)[..., : 2 * T]
    close(got.cpu().transpose(1, 2), ref)
    with pytest.raises(nat.NativeError, match="unsupported"):
        nat.call("fm_row_linear_packed_upsample", x.data_ptr(), B * T, 2048, wp.data_ptr(), N, T,
                 up.data_ptr(), got.data_ptr(), stream())


@pytest.mark.parametrize("B,L,C", [(1, 125, 512), (3, 7, 16), (2, 1, 512)])
def test_upsample_depthwise(B, L, C):
    g = torch.Generator().manual_seed(L)
    x = torch.randn(B, C, L, generator=g)
    w = torch.randn(C, 1, 4, generator=g)
    y = torch.empty(B, 2 * L, C, device=DEV)
    x_d, w_d = x.transpose(1, 2).contiguous().to(DEV), w.to(DEV)
    nat.call("fm_upsample_depthwise", x_d.data_ptr(), B, L, C, w_d.data_ptr(), 4, 2, y.data_ptr(),
             stream())
    torch.cuda.synchronize()
    want = causal_conv_transpose1d(x.double(), w.double(), None, 2, groups=C)
    close(y.cpu().transpose(1, 2), want, rel=1e-6)


def test_bad_arguments_are_rejected():
    with pytest.raises(nat.NativeError, match="bad argument"):
        nat.call("fm_layer_norm", None, None, None, 4, 8, 1e-5, None, stream())
    with pytest.raises(nat.NativeError, match="unsupported"):
        nat.call("fm_window_attention", 1, 8, 0, 0, 0, 1, 1, 1, 1, 1, 1, 12, 8, 1.0, 1, 8, stream())


def test_split_k_is_deterministic(ws):
    """Small-M, large-K GEMMs split K across the waves of a block and across
    blocks; both sums run in a fixed order, so repeated calls agree bit for bit."""
    g = torch.Generator().manual_seed(12)
    x = torch.randn(250, 8192, generator=g).to(DEV)
    w = (torch.randn(1024, 8192, generator=g) * 0.01).to(DEV)
    first = run_linear(x, w, ws=ws).clone()
    second = run_linear(x, w, ws=ws)
    assert torch.equal(first, second)
    close(first.cpu(), x.double().cpu() @ w.double().cpu().t())


@pytest.mark.parametrize("rows,k,n,x6", [
    (250, 8192, 512, False),    # 64x64 16x16-MFMA tiles split along K
    (125, 4096, 512, False),    # 32x32 tiles, K split inside the block and across blocks
    (12000, 1280, 256, True),   # 128x128 bf16x6 tiles split along K
    (2500, 2048, 512, True),    # 64x128 bf16x6 tiles split along K
])
def test_split_k_repeats_and_graph_replays(rows, k, n, x6, ws):
    """K-split GEMMs (partials in the shared workspace, summed in split order):
    back-to-back calls, calls of another split shape in between and hipGraph
    replays all give the same bits, and the LayerScale residual epilogue is
    applied once to the ordered sum."""
    g = torch.Generator().manual_seed(rows + k + n)
    x = torch.randn(rows, k, generator=g)
    w = torch.randn(n, k, generator=g) / math.sqrt(k)
    res = torch.randn(rows, n, generator=g)
    scale = torch.rand(n, generator=g) + 0.5
    xd, wd, rd, sd = x.to(DEV), w.to(DEV), res.to(DEV), scale.to(DEV)
    f = nat.EPI_RES_SCALE
    if x6:
        wd, f = with_planes(wd), f | nat.WEIGHTS_X6
    first = run_linear(xd, wd, f, res=rd, scale=sd, ws=ws).clone()
    prod = x.double() @ w.double().t()
    close(first.cpu(), res.double() + scale.double() * prod)
    other_x = torch.randn(250, 8192, generator=g).to(DEV)
    other_w = (torch.randn(512, 8192, generator=g) * 0.01).to(DEV)
    for _ in range(3):
        assert torch.equal(run_linear(xd, wd, f, res=rd, scale=sd, ws=ws), first)
        run_linear(other_x, other_w, ws=ws)
    out = torch.empty_like(first)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        nat.call("fm_linear", xd.data_ptr(), rows, k, wd.data_ptr(), n, f, rd.data_ptr(),
                 sd.data_ptr(), out.data_ptr(), ws.data_ptr(), WS_BYTES, stream())
    for _ in range(3):
        out.zero_()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, first)
        run_linear(other_x, other_w, ws=ws)


def test_gemm_plan_names_the_launched_kernel():
    """fm_gemm_last_plan reports the selection's kernel: the C2 dec.up4
    transposed conv (60000 x 256 x 256, weights with bf16x6 planes) takes the
    256x128 bf16x6 tile, one round of 470 tiles."""
    from fast_mimi_amd import MimiConfig, MimiModel

    rt = MimiModel(MimiConfig(), device=DEV, seed=0).runtime()
    op = rt.layer_op("dec.up4", 1, 240_000)
    op()
    torch.cuda.synchronize()
    assert nat.last_gemm_plan() == "gemm_x6d_kernel<256,128,8,1,2,false> tiles=470 splits=1"


@pytest.mark.parametrize("rows,k,n,flags", [(2000, 512, 1536, 0), (2500, 512, 1536, 0),
                                           (1500, 1024, 2048, 0), (2000, 512, 2048, nat.EPI_GELU)])
def test_x6_tile_choice_leaves_results_unchanged(rows, k, n, flags, ws):
    """Every bf16x6 tile accumulates an output element in the same order, so
    the tile picked for a grid never changes a result: rows computed in a
    grid of at most 256 128x128 tiles (64x128 tiles) equal, bit for bit, the
    same rows computed inside a grid twice as tall (192x128 or 128x128
    tiles)."""
    g = torch.Generator().manual_seed(rows + k + n)
    x = torch.randn(rows, k, generator=g).to(DEV)
    w = with_planes((torch.randn(n, k, generator=g) / math.sqrt(k)).to(DEV))
    f = flags | nat.WEIGHTS_X6
    small = torch.empty(rows, n, device=DEV)
    nat.call("fm_linear", x.data_ptr(), rows, k, w.data_ptr(), n, f, None, None, small.data_ptr(),
             ws.data_ptr(), WS_BYTES, stream())
    plan_small = nat.last_gemm_plan()
    x2 = torch.cat([x, x.flip(0)])
    big = torch.empty(2 * rows, n, device=DEV)
    nat.call("fm_linear", x2.data_ptr(), 2 * rows, k, w.data_ptr(), n, f, None, None, big.data_ptr(),
             ws.data_ptr(), WS_BYTES, stream())
    plan_big = nat.last_gemm_plan()
    torch.cuda.synchronize()
    assert "gemm_x6d_kernel<64,128" in plan_small and "splits=1" in plan_small, plan_small
    assert "gemm_x6d_kernel<64,128" not in plan_big and "splits=1" in plan_big, plan_big
    assert torch.equal(small, big[:rows])
    assert torch.equal(small.flip(0), big[rows:])


@pytest.mark.parametrize("n0,n1,off0,off1", [(240000 * 4, 8 * 250 * 8, 0, 0), (1, 17, 0, 0), (1000, 0, 3, 0),
                                           (4096 + 5, 333, 1, 7), (0, 64, 0, 0), (16 << 20, 12345, 0, 5)])
def test_copy_buffers(n0, n1, off0, off1):
    """fm_copy_buffers copies both byte ranges exactly (16-byte vectors when
    every pointer is aligned, bytes otherwise, zero sizes skipped) and writes
    nothing outside them."""
    g = torch.Generator().manual_seed(n0 + n1)
    src = [torch.randint(0, 256, (n + 16,), generator=g, dtype=torch.uint8).to(DEV) for n in (n0, n1)]
    dst = [torch.full((n + 32,), 0xA5, dtype=torch.uint8, device=DEV) for n in (n0, n1)]
    offs = (off0, off1)
    ptr = lambda t, o: t.data_ptr() + o
    nat.call("fm_copy_buffers", ptr(src[0], offs[0]), ptr(dst[0], offs[0]), n0,
             ptr(src[1], offs[1]), ptr(dst[1], offs[1]), n1, stream())
    torch.cuda.synchronize()
    for s_, d_, n, o in zip(src, dst, (n0, n1), offs):
        assert torch.equal(d_[o:o + n], s_[o:o + n])
        assert bool((d_[:o] == 0xA5).all()) and bool((d_[o + n:] == 0xA5).all())


@pytest.mark.parametrize("rows,per_seq,k,n,rope_cols,fused", [
    (2500, 2500, 512, 1536, 1024, True),   # C4 qkv: 64x128 tiles
    (4000, 250, 512, 1536, 1024, True),    # C3 qkv: 192x128 tiles, 16 sequences
    (16000, 250, 512, 1536, 1024, True),   # C5 qkv: 256x128 tiles
    (1100, 100, 512, 1536, 512, False),    # an FP32 tile: the GEMM, then fm_apply_rope
    (1500, 250, 2048, 512, 512, False),    # a split plan: likewise
])
def test_linear_rope_equals_linear_then_rope(rows, per_seq, k, n, rope_cols, fused, ws):
    """fm_linear_rope equals fm_linear followed by fm_apply_rope bit for bit:
    RoPE in the epilogue of an unsplit bf16x6 tile, else fm_linear's own
    plan and then the RoPE kernel (so the projection rounds the same)."""
    from fast_mimi_amd import MimiConfig
    from fast_mimi_amd.runtime import rope_tables

    g = torch.Generator().manual_seed(rows + k + n)
    x = torch.randn(rows, k, generator=g).to(DEV)
    w = with_planes((torch.randn(n, k, generator=g) / math.sqrt(k)).to(DEV))
    cos, sin = (t.to(DEV) for t in rope_tables(MimiConfig(), per_seq))
    want = torch.empty(rows, n, device=DEV)
    nat.call("fm_linear", x.data_ptr(), rows, k, w.data_ptr(), n, nat.WEIGHTS_X6, None, None,
             want.data_ptr(), ws.data_ptr(), WS_BYTES, stream())
    nat.call("fm_apply_rope", want.data_ptr(), rows, n, rope_cols, 64, cos.data_ptr(), sin.data_ptr(),
             per_seq, stream())
    got = torch.full((rows, n), float("nan"), device=DEV)
    nat.call("fm_linear_rope", x.data_ptr(), rows, k, w.data_ptr(), n, nat.WEIGHTS_X6, cos.data_ptr(),
             sin.data_ptr(), rope_cols, per_seq, got.data_ptr(), ws.data_ptr(), WS_BYTES, stream())
    plan = nat.last_gemm_plan()
    torch.cuda.synchronize()
    assert ("gemm_x6d_kernel" in plan and "splits=1" in plan) == fused, plan
    assert torch.equal(got, want)


def test_rvq_split_with_a_per_step_sized_workspace():
    """A workspace sized by fm_rvq_workspace_bytes alone (smaller than the
    one-launch chain needs at a few rows) takes the per-step launches: same
    codes, nothing written past the workspace."""
    B, T, nsem, nac, e, d = 1, 20, 1, 7, 2048, 256
    g = torch.Generator().manual_seed(5)
    n = nsem + nac
    emb, emb_t, norms = prepare_codebooks(torch.randn(n, e, d, generator=g) / 16, torch.ones(n, e))
    x = (torch.randn(B * T, 2 * d, generator=g) * 0.3).to(DEV)
    lib = nat.library()
    out = []
    for wsb in (2 * lib.fm_rvq_workspace_bytes(B * T, d, e), lib.fm_rvq_split_workspace_bytes(B * T, d, e)):
        guard = torch.full(((wsb + 3) // 4 + 4096,), 7.0, device=DEV)
        codes = torch.full((B, n, T), -1, dtype=torch.int64, device=DEV)
        nat.call("fm_rvq_encode_split", x.data_ptr(), 2 * d, B * T, T, d, e, nsem, nac, emb.data_ptr(),
                 emb_t.data_ptr(), norms.data_ptr(), codes.data_ptr(), n * T, guard.data_ptr(), wsb, stream())
        torch.cuda.synchronize()
        assert (guard[(wsb + 3) // 4:] == 7.0).all()
        out.append(codes.cpu())
    assert torch.equal(out[0], out[1])
