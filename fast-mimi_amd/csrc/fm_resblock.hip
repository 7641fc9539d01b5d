// Fused SEANet residual block (kadirnar/fast-mimi src/fast_mimi/model.py:947-971):
//
//   y = ELU?( x + conv1x1( ELU( conv_k3( ELU(x) ) + b1 ) ) + b2 )
//
// on channels-last x [batch, L, C] with causal (left) zero padding of 2 and
// hidden width C/2.  A block owns 32-row tiles of one batch item.  ELU(x) for
// rows t0-2 .. t0+BM-1 (the causal halo included) is staged in LDS once; the
// k3 convolution reads its three taps as row-shifted views of that tile, so
// the input is read from HBM once instead of once per tap.  The hidden
// activations never leave LDS; the 1x1 convolution adds the raw residual
// (read once, coalesced) and the block's trailing ELU in its epilogue.  Both
// GEMMs run on FP32 MFMA with the k-permuted 16-byte fragment reads of the
// main GEMM engine (k-slot of lane half h at step 4q+e carries k = 16h + 4q +
// e).  Weights are the packed conv layout: W1^T [C/2][3C] (k = tap*C + c_in)
// and W2^T [C][C/2].

#include "fm_common.h"

namespace {

constexpr int NT = 256;

// ---------------------------------------------------------------------------
// C = 64 residual block as a persistent kernel.  The block's weights are
// staged once in LDS as MFMA B-fragment rows (W1^T [32][192], W2^T [64][32]),
// shared by the 12 waves.  Each wave then takes 32-row tiles in a grid-stride
// loop with no block-level barrier: stage ELU(x) rows t0-2 .. t0+31 in its own
// LDS slot, issue the residual rows of this tile (they land during the
// MFMAs), k3 conv (96 MFMAs in two chains, taps as row-shifted views), hidden
// = ELU(acc + b1) into the same slot, 1x1 conv (32 MFMAs), then the output
// tile goes back through the slot so the epilogue (bias, raw residual, ELU)
// runs on float4 runs.  One 9 KB slot per wave keeps three waves per SIMD,
// which overlap one tile's memory and ELU work with the others' MFMAs.
// MFMA k-slots: lane half h at step 4q+e carries k = 96h + 4q + e (k3 conv,
// k = tap*64 + c_in) or 16h + 4q + e (1x1 conv).
// WAVE_IN: x is the 1-channel waveform [batch][L] and the block's input is
// the encoder's first conv, x64[t][c] = b0[c] + sum_j w0[c][j] * wav[t-6+j]
// (j = 0..6, zero outside the waveform; the FMA order of conv_cin1_kernel).
// Each wave stages the 40 samples its tile needs and every lane forms its
// input rows (ELU'd into the slot) and residual rows in registers, so the
// 64-channel activation never goes through HBM.
// WAVE_OUT: the block feeds the decoder's last conv (64 -> 1, kernel 3): the
// output rows go back into the slot and each row's three tap dot products
// w3[j] . y[t] are stored (float4 per row, D[b][t] = {d0, d1, d2, 0}) instead
// of y; conv3_finish_kernel then sums the taps of rows t-2, t-1, t.
constexpr int R64_WAVES = 12;
constexpr int R64_PE = 68;   // pitch of the ELU(x) / output tile rows
constexpr int R64_PH = 36;   // pitch of the hidden tile rows
constexpr int R64_SLOT = 34 * R64_PE;  // the hidden tile reuses the ELU(x) rows
constexpr int R64_P1 = 196;  // W1^T row pitch (4 mod 32: conflict-free 16-byte reads)
constexpr int R64_P2 = 36;   // W2^T row pitch
constexpr int R64_WIN = 40;  // waveform samples per tile (WAVE_IN)
constexpr int R64_WINP = 44; // their per-wave LDS pitch (reads reach index 41)

template <bool WAVE_IN, bool WAVE_OUT>
__global__ __launch_bounds__(64 * R64_WAVES) void resblock64_kernel(
    const float* __restrict__ x, int batch, int L, const float* __restrict__ w1,
    const float* __restrict__ b1, const float* __restrict__ w2, const float* __restrict__ b2,
    int elu_out, float* __restrict__ y, const float* __restrict__ w0, const float* __restrict__ b0) {
  constexpr int C = 64, HC = 32;
  constexpr int WIN_F = WAVE_IN ? R64_WAVES * R64_WINP : 0;
  constexpr int W3_F = WAVE_OUT ? 3 * 64 : 0;
  __shared__ __attribute__((aligned(16))) float smem[R64_WAVES * R64_SLOT + 32 * R64_P1 + 64 * R64_P2 + WIN_F + W3_F];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  float* E = smem + wave * R64_SLOT;   // [34][68] ELU(x); later the [32][68] output tile
  float* H = E;                        // [32][36] hidden, over the consumed ELU(x) rows
  float* W1s = smem + R64_WAVES * R64_SLOT;
  float* W2s = W1s + 32 * R64_P1;
  float* Win = W2s + 64 * R64_P2 + wave * R64_WINP;  // WAVE_IN: this wave's samples t0-8 .. t0+31
  float* W3s = W2s + 64 * R64_P2 + WIN_F;             // WAVE_OUT: w3 [3][64] (w0 carries it)
  if constexpr (WAVE_OUT) {
    if (threadIdx.x < 3 * 64) W3s[threadIdx.x] = w0[threadIdx.x];
  }

  for (int i = threadIdx.x; i < 32 * 48; i += 64 * R64_WAVES) {
    const int r = i / 48, c4 = (i % 48) * 4;
    *reinterpret_cast<floatx4*>(W1s + r * R64_P1 + c4) = *reinterpret_cast<const floatx4*>(w1 + r * 192 + c4);
  }
  for (int i = threadIdx.x; i < 64 * 8; i += 64 * R64_WAVES) {
    const int r = i / 8, c4 = (i % 8) * 4;
    *reinterpret_cast<floatx4*>(W2s + r * R64_P2 + c4) = *reinterpret_cast<const floatx4*>(w2 + r * HC + c4);
  }
  const float bias1 = b1[lcol];
  // WAVE_IN: the first conv's weights for this lane's four channels.
  const int cg4 = (lane & 15) * 4, q = lane >> 4;
  float w0r[4][7], b0r[4];
  if constexpr (WAVE_IN && !WAVE_OUT) {
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b0r[e] = b0[cg4 + e];
#pragma unroll
      for (int j = 0; j < 7; ++j) w0r[e][j] = w0[(cg4 + e) * 7 + j];
    }
  }
  __syncthreads();

  const int tpb = (L + 31) / 32;
  const long tiles = (long)batch * tpb;
  const long stride = (long)gridDim.x * R64_WAVES;
  long tile = (long)blockIdx.x * R64_WAVES + wave;

  // x rows t0-2 .. t0+31 of a tile: 544 float4 chunks, 9 per lane (chunk c = lane + 64u).
  floatx4 xv[9];
  unsigned xok = 0;
  float wv = 0.0f;  // WAVE_IN: sample t0 - 8 + lane of the tile (lanes < 40)
  auto load_x = [&](long tl) {
    const int b = (int)(tl / tpb), t0 = (int)(tl % tpb) * 32;
    if constexpr (WAVE_IN) {
      const int t = t0 - 8 + lane;
      wv = (lane < R64_WIN && t >= 0 && t < L) ? x[(long)b * L + t] : 0.0f;
      return;
    }
    const float* xb = x + (long)b * L * C;
    xok = 0;
#pragma unroll
    for (int u = 0; u < 9; ++u) {
      const int c = lane + 64 * u;
      const int t = t0 - 2 + c / 16;
      const bool ok = c < 544 && t >= 0 && t < L;
      xv[u] = *reinterpret_cast<const floatx4*>(xb + (long)min(max(t, 0), L - 1) * C + (c % 16) * 4);
      xok |= (unsigned)ok << u;
    }
  };
  // The 1-sample waveform window is prefetched a tile ahead; 64-channel rows
  // are loaded at the start of their own tile (three waves per SIMD cover the
  // latency, and a second register set would not fit their budget).
  if (WAVE_IN && tile < tiles) load_x(tile);
  for (; tile < tiles; tile += stride) {
    const int b = (int)(tile / tpb), t0 = (int)(tile % tpb) * 32;
    if constexpr (!WAVE_IN) load_x(tile);
    floatx4 rv[8];
    if constexpr (WAVE_IN) {
      // Samples t0-8 .. t0+31 into the wave's window; lane (q, cg) then needs
      // samples q .. q+38 of it.  Staged row rr (t = t0-2+rr) reads
      // window[rr .. rr+6]; the lane forms rows rr = q + 4u + 2 (u < 8: the
      // block's own rows t0 + q + 4u, which are also its residual rows) and,
      // for q < 2, the causal halo row rr = q.
      if (lane < R64_WIN) Win[lane] = wv;
      wave_lds_fence();
      if (tile + stride < tiles) load_x(tile + stride);
      float s[39];
#pragma unroll
      for (int i = 0; i < 39; ++i) s[i] = Win[q + i];
      auto conv0 = [&](int base) {
        floatx4 v;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float acc = b0r[e];
#pragma unroll
          for (int j = 0; j < 7; ++j) acc = fmaf(w0r[e][j], s[base + j], acc);
          v[e] = acc;
        }
        return v;
      };
      auto stage = [&](int rr, floatx4 v) {
        *reinterpret_cast<floatx4*>(E + rr * R64_PE + cg4) =
            floatx4{fm_elu(v[0]), fm_elu(v[1]), fm_elu(v[2]), fm_elu(v[3])};
      };
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        rv[u] = conv0(4 * u + 2);
        stage(q + 4 * u + 2, t0 + q + 4 * u < L ? rv[u] : floatx4{0.0f, 0.0f, 0.0f, 0.0f});
      }
      if (q < 2) stage(q, t0 - 2 + q >= 0 ? conv0(0) : floatx4{0.0f, 0.0f, 0.0f, 0.0f});
    } else {
      const float* xb = x + (long)b * L * C;
      // ELU(x) into the slot (zero outside the sequence: the causal zero padding).
#pragma unroll
      for (int u = 0; u < 9; ++u) {
        const int c = lane + 64 * u;
        if (c >= 544) continue;
        floatx4 v = ((xok >> u) & 1) ? xv[u] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        *reinterpret_cast<floatx4*>(E + (c / 16) * R64_PE + (c % 16) * 4) =
            floatx4{fm_elu(v[0]), fm_elu(v[1]), fm_elu(v[2]), fm_elu(v[3])};
      }
      // Raw residual rows t0 .. t0+31 (chunk c = lane + 64u, 8 per lane) and the
      // next tile's input rows: both in flight during this tile's MFMAs.
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int c = lane + 64 * u;
        rv[u] = *reinterpret_cast<const floatx4*>(xb + (long)min(t0 + c / 16, L - 1) * C + (c % 16) * 4);
      }
    }
    wave_lds_fence();

    // k3 conv: rows = positions, columns = hidden channels; two chains.
    floatx16 acc1[2];
#pragma unroll
    for (int c = 0; c < 2; ++c)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc1[c][r] = 0.0f;
#pragma unroll
    for (int q = 0; q < 24; ++q) {
      const int k0 = 96 * h + 4 * q;
      const floatx4 a = *reinterpret_cast<const floatx4*>(E + (lcol + k0 / 64) * R64_PE + k0 % 64);
      const floatx4 wq = *reinterpret_cast<const floatx4*>(W1s + lcol * R64_P1 + k0);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc1[q & 1] = fm_mfma32(a[e], wq[e], acc1[q & 1]);
    }
    wave_lds_fence();  // the k3 conv's reads of the ELU(x) rows are done before H overwrites them
#pragma unroll
    for (int r = 0; r < 16; ++r)
      H[fm_mfma32_row(r, lane) * R64_PH + lcol] = fm_elu(__fadd_rn(__fadd_rn(acc1[0][r], acc1[1][r]), bias1));
    wave_lds_fence();

    // 1x1 conv: columns = output channels (two 32-wide tiles).
    floatx16 acc2[2];
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc2[j][r] = 0.0f;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(H + lcol * R64_PH + 16 * h + 4 * q);
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const floatx4 wq = *reinterpret_cast<const floatx4*>(W2s + (j * 32 + lcol) * R64_P2 + 16 * h + 4 * q);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc2[j] = fm_mfma32(a[e], wq[e], acc2[j]);
      }
    }
    // Output tile through LDS, over H once the 1x1 conv has read it.
    wave_lds_fence();
#pragma unroll
    for (int j = 0; j < 2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) E[fm_mfma32_row(r, lane) * R64_PE + j * 32 + lcol] = acc2[j][r];
    wave_lds_fence();
    float* yb = y + (long)b * L * C;
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = lane + 64 * u;
      const int r = c / 16, c4 = (c % 16) * 4;
      const floatx4 acc = *reinterpret_cast<const floatx4*>(E + r * R64_PE + c4);
      const floatx4 bb = *reinterpret_cast<const floatx4*>(b2 + c4);
      floatx4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[e] = __fadd_rn(rv[u][e], __fadd_rn(acc[e], bb[e]));
        if (elu_out) v[e] = fm_elu(v[e]);
      }
      if constexpr (WAVE_OUT) {
        *reinterpret_cast<floatx4*>(E + r * R64_PE + c4) = v;
      } else {
        if (t0 + r < L) *reinterpret_cast<floatx4*>(yb + (long)(t0 + r) * C + c4) = v;
      }
    }
    if constexpr (WAVE_OUT) {
      // Row r = lane % 32, channel half hh = lane / 32: the three tap dot
      // products over 32 channels, then half 0 + half 1.
      wave_lds_fence();
      const int r = lane & 31, hh = lane >> 5;
      float d[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int c = 0; c < 32; c += 4) {
        const floatx4 v = *reinterpret_cast<const floatx4*>(E + r * R64_PE + 32 * hh + c);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const floatx4 wj = *reinterpret_cast<const floatx4*>(W3s + j * 64 + 32 * hh + c);
          d[j] = fmaf(wj[0], v[0], d[j]);
          d[j] = fmaf(wj[1], v[1], d[j]);
          d[j] = fmaf(wj[2], v[2], d[j]);
          d[j] = fmaf(wj[3], v[3], d[j]);
        }
      }
      floatx4 o;
#pragma unroll
      for (int j = 0; j < 3; ++j) o[j] = __fadd_rn(d[j], __shfl_xor(d[j], 32, 64));
      o[3] = 0.0f;
      if (hh == 0 && t0 + r < L) *reinterpret_cast<floatx4*>(y + ((long)b * L + t0 + r) * 4) = o;
    }
    wave_lds_fence();  // the slot is rewritten by the next tile
  }
}

// out[b][t] = ((d0[t-2] + d1[t-1]) + d2[t]) + bias for t < y_len, with the
// per-row tap products D of resblock64_kernel<*, true> (rows < 0 are zero).
__global__ __launch_bounds__(256) void conv3_finish_kernel(const float* __restrict__ D, int L,
                                                           int y_len, const float* __restrict__ bias,
                                                           float* __restrict__ out) {
  const long b = blockIdx.y;
  const int t = blockIdx.x * 256 + threadIdx.x;
  if (t >= y_len) return;
  const float* Db = D + b * (long)L * 4;
  const float d0 = t >= 2 ? Db[(long)(t - 2) * 4 + 0] : 0.0f;
  const float d1 = t >= 1 ? Db[(long)(t - 1) * 4 + 1] : 0.0f;
  float s = __fadd_rn(__fadd_rn(d0, d1), Db[(long)t * 4 + 2]);
  if (bias) s = __fadd_rn(s, bias[0]);
  out[b * y_len + t] = s;
}

// ---------------------------------------------------------------------------
// Residual block with register-streamed weights.  Waves form WM x (4 / WM):
// wave (wr, wc) owns output rows wr*32 .. +31 of the block, hidden columns
// wc*HC/WN .. (one 32-wide MFMA tile) and output columns wc*C/WN .. (two
// 32-wide tiles).  A wave's weight fragments are read straight from the
// row-major W1^T [HC][3C] / W2^T [C][HC] (L2-resident, 16-byte k-permuted
// lane reads) into a PD-deep register ring, so the k-loops have no block
// barrier and LDS holds only ELU(x) with its causal halo and the hidden tile
// (~52 KB: three blocks per CU).  One barrier separates the two convs.  In
// the k3 conv the A fragments of the next 32-k step are read from LDS while
// the current step's MFMAs run.
template <int C, int BM, int WM, int PD>
__global__ __launch_bounds__(NT, 3) void resblock_direct_kernel(
    const float* __restrict__ x, int L, const float* __restrict__ w1, const float* __restrict__ b1,
    const float* __restrict__ w2, const float* __restrict__ b2, int elu_out, float* __restrict__ y) {
  constexpr int WN = 4 / WM, HC = C / 2, K1 = 3 * C;
  constexpr int PX = C + 4, PH = HC + 4;
  constexpr int T1 = K1 / 32, T2 = HC / 32, FN2 = 2;
  constexpr int T = T1 + T2 * FN2;
  static_assert(BM == 32 * WM && HC / WN == 32 && C / WN == 32 * FN2, "wave tiling");
  __shared__ __attribute__((aligned(16))) float Xe[(BM + 2) * PX];
  __shared__ __attribute__((aligned(16))) float Hs[BM * PH];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  const int wr = wave / WN, wc = wave % WN;
  const long b = blockIdx.y;
  const int t0 = blockIdx.x * BM;
  const float* xb = x + b * (long)L * C;
  // Interior blocks (halo and rows inside the sequence) address every row
  // through raw buffers: a lane offset plus compile-time row offsets, no
  // per-element bounds checks.  Edge blocks take the checked path.
  // Byte counts in 64-bit: the raw buffers are only used (and only sized)
  // when a batch item's activation fits a 32-bit offset.
  const long act_bytes = (long)L * C * 4;
  const bool fast = t0 >= 2 && t0 + BM <= L && act_bytes <= 0x7fffffffL;
  const __amdgpu_buffer_rsrc_t rx = fm_buffer(xb, fast ? (int)act_bytes : 0);
  const __amdgpu_buffer_rsrc_t ry = fm_buffer(y + b * (long)L * C, fast ? (int)act_bytes : 0);
  const int vrow = ((t0 + wr * 32 + 4 * h) * C + wc * 64 + lcol) * 4;  // this lane's first output element
  auto row_off = [&](int r, int j) { return ((8 * (r >> 2) + (r & 3)) * C + j * 32) * 4; };

  // Input rows first (the critical path), weight ring right behind them.
  constexpr int CH = (BM + 2) * C / 4, U = (CH + NT - 1) / NT;
  floatx4 xv[U];
  if (fast) {
    // The tile's rows t0-2 .. t0+BM-1 are one contiguous run of CH chunks.
    const int vo = ((t0 - 2) * C + 4 * tid) * 4;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xv[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (u + 1 < U || tid + u * NT < CH) xv[u] = fm_buf_load4(rx, vo, u * NT * 16);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = tid + u * NT;
      const int r = c / (C / 4), k = (c % (C / 4)) * 4;
      const int t = t0 - 2 + r;
      xv[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (c < CH && t >= 0 && t < L) xv[u] = *reinterpret_cast<const floatx4*>(xb + (long)t * C + k);
    }
  }
  const float* w1p = w1 + (long)(wc * 32 + lcol) * K1 + 16 * h;
  const float* w2p = w2 + (long)(wc * 64 + lcol) * HC + 16 * h;
  floatx4 ring[PD][4];
  auto load_unit = [&](int u, floatx4 (&d)[4]) {
    const float* src;
    if (u < T1) {
      src = w1p + u * 32;
    } else {
      const int v = u - T1, kt = v / FN2, j = v % FN2;
      src = w2p + (long)j * 32 * HC + kt * 32;
    }
#pragma unroll
    for (int q = 0; q < 4; ++q) d[q] = *reinterpret_cast<const floatx4*>(src + 4 * q);
  };
#pragma unroll
  for (int d = 0; d < PD; ++d) load_unit(d, ring[d]);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = tid + u * NT;
    if (c >= CH) continue;
    const int r = c / (C / 4), k = (c % (C / 4)) * 4;
    *reinterpret_cast<floatx4*>(&Xe[r * PX + k]) =
        floatx4{fm_elu(xv[u].x), fm_elu(xv[u].y), fm_elu(xv[u].z), fm_elu(xv[u].w)};
  }
  __syncthreads();

  const int arow = wr * 32 + lcol;
  // Stage-1 A fragments of k-step u: the row-shifted view of tap u*32 / C.
  auto load_a1 = [&](int u, floatx4 (&a)[4]) {
    const int kk0 = u * 32, tap = kk0 / C, ci0 = kk0 % C;
#pragma unroll
    for (int q = 0; q < 4; ++q)
      a[q] = *reinterpret_cast<const floatx4*>(&Xe[(arow + tap) * PX + ci0 + 16 * h + 4 * q]);
  };
  auto load_a2 = [&](int kt, floatx4 (&a)[4]) {
#pragma unroll
    for (int q = 0; q < 4; ++q)
      a[q] = *reinterpret_cast<const floatx4*>(&Hs[arow * PH + kt * 32 + 16 * h + 4 * q]);
  };

  // conv k3: two accumulator chains (even / odd 4-k steps).
  floatx16 acc1[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc1[i][r] = 0.0f;
  floatx4 a[2][4];
  load_a1(0, a[0]);
#pragma unroll
  for (int u = 0; u < T1; ++u) {
    if (u + 1 < T1) load_a1(u + 1, a[(u + 1) & 1]);
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc1[q & 1] = fm_mfma32(a[u & 1][q][e], ring[u % PD][q][e], acc1[q & 1]);
    // Refill the slot just consumed; the barrier keeps the compiler from
    // sinking the loads to their use (which serialises them).
    if (u + PD < T) load_unit(u + PD, ring[u % PD]);
    __builtin_amdgcn_sched_barrier(0);
  }
  {
    const int n = wc * 32 + lcol;
    const float bias = b1[n];
#pragma unroll
    for (int r = 0; r < 16; ++r)
      Hs[(wr * 32 + fm_mfma32_row(r, lane)) * PH + n] =
          fm_elu(__fadd_rn(__fadd_rn(acc1[0][r], acc1[1][r]), bias));
  }
  __syncthreads();

  // Residual rows land during the 1x1 conv.
  float* yb = y + b * (long)L * C;
  float rv[FN2][16];
  if (fast) {
#pragma unroll
    for (int j = 0; j < FN2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) rv[j][r] = fm_buf_load1(rx, vrow, row_off(r, j));
  } else {
#pragma unroll
    for (int j = 0; j < FN2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = min(t0 + wr * 32 + fm_mfma32_row(r, lane), L - 1);
        rv[j][r] = xb[(long)t * C + wc * 64 + j * 32 + lcol];
      }
  }
  floatx16 acc2[FN2];
#pragma unroll
  for (int j = 0; j < FN2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc2[j][r] = 0.0f;
#pragma unroll
  for (int kt = 0; kt < T2; ++kt) {
    load_a2(kt, a[0]);
#pragma unroll
    for (int j = 0; j < FN2; ++j) {
      const int u = T1 + kt * FN2 + j;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e) acc2[j] = fm_mfma32(a[0][q][e], ring[u % PD][q][e], acc2[j]);
      if (u + PD < T) load_unit(u + PD, ring[u % PD]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
#pragma unroll
  for (int j = 0; j < FN2; ++j) {
    const int n = wc * 64 + j * 32 + lcol;
    const float bias = b2[n];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = t0 + wr * 32 + fm_mfma32_row(r, lane);
      float v = __fadd_rn(rv[j][r], __fadd_rn(acc2[j][r], bias));
      if (elu_out) v = fm_elu(v);
      if (fast) {
        fm_buf_store1(v, ry, vrow, row_off(r, j));
      } else if (t < L) {
        yb[(long)t * C + n] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------
// The C = 128 / 256 residual block on the bf16 matrix cores (bf16x6: every
// FP32 operand is three round-to-nearest bf16 pieces and each product is the
// six cross terms of order <= 2, accumulated in FP32; the error stays at FP32
// level).  The block layout is resblock_direct_kernel's: wave (wr, wc) owns
// positions wr*32 .. +31, hidden channels wc*32 .. +31 and output channels
// wc*64 .. +63; weights stream from L2 into a PD-deep register ring.
// ELU(x) of rows t0-2 .. t0+BM-1 is split once as it is staged and kept as
// three bf16 planes [BM+2][C] whose 16-byte chunks are XOR-swizzled by
// (row & 7), so the row-shifted tap views read conflict-free.  The k3 conv is
// computed transposed (hidden x positions: the weight planes are the A
// operand) so each lane ends with four consecutive hidden channels of one
// position, split and written as 8-byte pieces into hidden planes [BM][C/2]
// laid over the consumed ELU(x) planes.  The 1x1 conv reads them as A
// fragments.  Weights are the packed W^T followed by their planes in k16-tile
// order [3][K/16][N][16] (fm_split_weights).  Both operands use the same k
// order: in a 32-deep k unit, MFMA step s of lane half h covers k = 16s + 8h
// .. +7, so a wave's weight fragment (32 rows x 16 k) is one contiguous 1 KB
// run (a [3][N][K] row-major layout spreads it over 32 cache lines, which the
// per-CU address path, not the MFMAs, then limits: 1.55x slower).
template <int C, int BM, int WM, int PD, bool WAVE_IN, bool WAVE_OUT, bool FAST_ACT = false>
__global__ __launch_bounds__(NT, 3) void resblock_x6_kernel(
    const float* __restrict__ x, int L, const __bf16* __restrict__ w1x, const float* __restrict__ b1,
    const __bf16* __restrict__ w2x, const float* __restrict__ b2, int elu_out, float* __restrict__ y,
    const float* __restrict__ w0, const float* __restrict__ b0) {
  constexpr int WN = 4 / WM, HC = C / 2, K1 = 3 * C;
  constexpr int XR = BM + 2, XPLANE = XR * C * 2, HPLANE = BM * HC * 2;
  constexpr int T1 = K1 / 32, T2 = HC / 32, FN2 = 2;
  constexpr int T = T1 + T2 * FN2;
  static_assert(BM == 32 * WM && HC / WN == 32 && C / WN == 32 * FN2, "wave tiling");
  static_assert(3 * HPLANE <= 3 * XPLANE, "hidden planes fit over the ELU(x) planes");
  static_assert(!(WAVE_IN || WAVE_OUT) || (C == 64 && WM == 4), "waveform ends: one wave per 32 rows x 64 channels");
  static_assert(!WAVE_OUT || 4 * 32 * 68 * 4 <= 3 * XPLANE, "output tiles fit");
  auto act = [](float v) { return FAST_ACT ? fm_elu_exp(v) : fm_elu(v); };
  __shared__ __attribute__((aligned(16))) char smem[3 * XPLANE];
  __shared__ float wins[WAVE_IN ? BM + 8 : 1];  // WAVE_IN: waveform samples t0-8 .. t0+BM-1

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  const int wr = wave / WN, wc = wave % WN;
  const long b = blockIdx.y;
  const int t0 = blockIdx.x * BM;
  // WAVE_IN: x is the waveform [batch][L] and the block input is the first
  // conv of the encoder, x64[t][c] = b0[c] + sum_j w0[c][j] wav[t-6+j]
  // (w0 [64][7], zero outside the waveform; the FMA order of
  // conv_cin1_kernel), formed for the staged rows and again for the
  // residual.  WAVE_OUT: y receives per row the three tap products of the
  // decoder's last conv (w0 = w3 [3][64]) instead of the block output.
  const float* xb = x + b * (long)L * (WAVE_IN ? 1 : C);
  const long act_bytes = (long)L * C * 4;  // 64-bit; see resblock_x6_kernel
  const bool fast = t0 >= 2 && t0 + BM <= L && act_bytes <= 0x7fffffffL;
  const __amdgpu_buffer_rsrc_t rx = fm_buffer(xb, fast ? (int)((long)L * (WAVE_IN ? 1 : C) * 4) : 0);
  const __amdgpu_buffer_rsrc_t ry = fm_buffer(y + b * (long)L * C, fast ? (int)act_bytes : 0);
  const int vrow = ((t0 + wr * 32 + 4 * h) * C + wc * 64 + lcol) * 4;
  auto row_off = [&](int r, int j) { return ((8 * (r >> 2) + (r & 3)) * C + j * 32) * 4; };
  // Byte offset of 16-byte chunk c of row r in a plane of `pitch`-byte rows
  // (chunks XOR-swizzled by the row within groups of up to 8 chunks).
  auto chunk = [](int r, int c, int pitch) {
    const int m = (pitch >> 4) < 8 ? (pitch >> 4) - 1 : 7;
    return r * pitch + ((c ^ (r & m)) << 4);
  };

  constexpr int CH = XR * C / 4, U = (CH + NT - 1) / NT;
  floatx4 xv[U];
  auto conv0 = [&](int c, int i0) {  // x64 at channel c from window samples i0 .. i0+6
    float acc = b0[c];
#pragma unroll
    for (int j = 0; j < 7; ++j) acc = fmaf(w0[c * 7 + j], wins[i0 + j], acc);
    return acc;
  };
  if constexpr (WAVE_IN) {
    for (int i = tid; i < BM + 8; i += NT) {
      const int t = t0 - 8 + i;
      wins[i] = (t >= 0 && t < L) ? xb[t] : 0.0f;
    }
    __syncthreads();
    // Staged row r (t = t0-2+r) reads samples t-6 .. t: window r .. r+6.
    const int k = (tid % (C / 4)) * 4;
    float w0r[4][7], b0r[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      b0r[e] = b0[k + e];
#pragma unroll
      for (int j = 0; j < 7; ++j) w0r[e][j] = w0[(k + e) * 7 + j];
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = tid + u * NT;
      const int r = c / (C / 4), t = t0 - 2 + r;
      xv[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (c < CH && t >= 0 && t < L) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          float acc = b0r[e];
#pragma unroll
          for (int j = 0; j < 7; ++j) acc = fmaf(w0r[e][j], wins[r + j], acc);
          xv[u][e] = acc;
        }
      }
    }
  } else if (fast) {
    const int vo = ((t0 - 2) * C + 4 * tid) * 4;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      xv[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (u + 1 < U || tid + u * NT < CH) xv[u] = fm_buf_load4(rx, vo, u * NT * 16);
    }
  } else {
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = tid + u * NT;
      const int r = c / (C / 4), k = (c % (C / 4)) * 4;
      const int t = t0 - 2 + r;
      xv[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (c < CH && t >= 0 && t < L) xv[u] = *reinterpret_cast<const floatx4*>(xb + (long)t * C + k);
    }
  }
  // Weight ring: unit u is 32 k of one 32-row weight slice, three planes,
  // two MFMA steps each.
  // Weight fragments through buffer resources: the lane's offset is fixed,
  // each unit's place in the planes is a scalar offset, so the streamed
  // loads take no vector address arithmetic.
  const __amdgpu_buffer_rsrc_t rw1 = fm_buffer(w1x, 3 * HC * K1 * 2);
  const __amdgpu_buffer_rsrc_t rw2 = fm_buffer(w2x, 3 * C * HC * 2);
  const int w1v = ((wc * 32 + lcol) * 16 + 8 * h) * 2, w2v = ((wc * 64 + lcol) * 16 + 8 * h) * 2;
  bf16x8 ring[PD][3][2];
  auto load_unit = [&](int u, bf16x8 (&d)[3][2]) {
    int base, plane;  // elements
    if (u < T1) {
      base = u * 2 * HC * 16;
      plane = HC * K1;
    } else {
      const int v = u - T1, kt = v / FN2, j = v % FN2;
      base = (j * 32 + kt * 2 * C) * 16;
      plane = C * HC;
    }
    const int tile = u < T1 ? HC * 16 : C * 16;  // elements per k16 tile of a plane
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        const int soff = (base + pl * plane + s * tile) * 2;
        d[pl][s] = __builtin_bit_cast(bf16x8, u < T1 ? fm_buf_load4(rw1, w1v, soff) : fm_buf_load4(rw2, w2v, soff));
      }
  };
#pragma unroll
  for (int d = 0; d < PD; ++d) load_unit(d, ring[d]);
#pragma unroll
  for (int u = 0; u < U; ++u) {
    const int c = tid + u * NT;
    if (c >= CH) continue;
    const int r = c / (C / 4), k = (c % (C / 4)) * 4;
    bf16x4 p0, p1, p2;
    split3(floatx4{act(xv[u].x), act(xv[u].y), act(xv[u].z), act(xv[u].w)}, p0, p1, p2);
    char* dst = smem + chunk(r, k >> 3, C * 2) + (k & 4) * 2;
    *reinterpret_cast<bf16x4*>(dst) = p0;
    *reinterpret_cast<bf16x4*>(dst + XPLANE) = p1;
    *reinterpret_cast<bf16x4*>(dst + 2 * XPLANE) = p2;
  }
  __syncthreads();

  // k3 conv, transposed: acc[hidden][position].  The B fragments (ELU(x)
  // planes) of the next unit are read while the current unit's MFMAs run.
  const int prow = wr * 32 + lcol;
  auto load_x = [&](int u, bf16x8 (&a)[3][2]) {
    const int kk0 = u * 32, tap = kk0 / C, c0 = (kk0 % C) / 8 + h;
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        a[pl][s] = *reinterpret_cast<const bf16x8*>(smem + pl * XPLANE + chunk(prow + tap, c0 + 2 * s, C * 2));
  };
  floatx16 acc1[2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc1[i][r] = 0.0f;
  bf16x8 xf[2][3][2];
  load_x(0, xf[0]);
#pragma unroll
  for (int u = 0; u < T1; ++u) {
    if (u + 1 < T1) load_x(u + 1, xf[(u + 1) & 1]);
    const bf16x8(&w)[3][2] = ring[u % PD];
    const bf16x8(&a)[3][2] = xf[u & 1];
#pragma unroll
    for (int s = 0; s < 2; ++s) {
      acc1[0] = fm_mfma32_bf16(w[1][s], a[1][s], acc1[0]);
      acc1[1] = fm_mfma32_bf16(w[2][s], a[0][s], acc1[1]);
      acc1[0] = fm_mfma32_bf16(w[1][s], a[0][s], acc1[0]);
      acc1[1] = fm_mfma32_bf16(w[0][s], a[2][s], acc1[1]);
      acc1[0] = fm_mfma32_bf16(w[0][s], a[1][s], acc1[0]);
      acc1[1] = fm_mfma32_bf16(w[0][s], a[0][s], acc1[1]);
    }
    if (u + PD < T) load_unit(u + PD, ring[u % PD]);
    __builtin_amdgcn_sched_barrier(0);
  }
  __syncthreads();  // every wave is done with the ELU(x) planes
  {
    // Lane: position prow, hidden channels wc*32 + 8g + 4h .. +3 (g = 0..3).
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const floatx4 bb = *reinterpret_cast<const floatx4*>(b1 + wc * 32 + 8 * g + 4 * h);
      floatx4 v;
#pragma unroll
      for (int e = 0; e < 4; ++e) v[e] = act(__fadd_rn(__fadd_rn(acc1[0][4 * g + e], acc1[1][4 * g + e]), bb[e]));
      bf16x4 p0, p1, p2;
      split3(v, p0, p1, p2);
      char* dst = smem + chunk(prow, wc * 4 + g, HC * 2) + 8 * h;
      *reinterpret_cast<bf16x4*>(dst) = p0;
      *reinterpret_cast<bf16x4*>(dst + HPLANE) = p1;
      *reinterpret_cast<bf16x4*>(dst + 2 * HPLANE) = p2;
    }
  }
  __syncthreads();

  float* yb = y + b * (long)L * C;
  float rv[FN2][16];
  if constexpr (WAVE_IN) {
    // Row rr = wr*32 + fm_mfma32_row(r, lane) (t = t0 + rr) reads window rr+2 .. rr+8.
#pragma unroll
    for (int j = 0; j < FN2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) rv[j][r] = conv0(wc * 64 + j * 32 + lcol, wr * 32 + fm_mfma32_row(r, lane) + 2);
  } else if (fast) {
#pragma unroll
    for (int j = 0; j < FN2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) rv[j][r] = fm_buf_load1(rx, vrow, row_off(r, j));
  } else {
#pragma unroll
    for (int j = 0; j < FN2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = min(t0 + wr * 32 + fm_mfma32_row(r, lane), L - 1);
        rv[j][r] = xb[(long)t * C + wc * 64 + j * 32 + lcol];
      }
  }
  // 1x1 conv: acc[position][output channel], two 32-wide column tiles.
  floatx16 acc2[FN2];
#pragma unroll
  for (int j = 0; j < FN2; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc2[j][r] = 0.0f;
#pragma unroll
  for (int kt = 0; kt < T2; ++kt) {
    bf16x8 a[3][2];
#pragma unroll
    for (int pl = 0; pl < 3; ++pl)
#pragma unroll
      for (int s = 0; s < 2; ++s)
        a[pl][s] = *reinterpret_cast<const bf16x8*>(smem + pl * HPLANE + chunk(prow, kt * 4 + 2 * s + h, HC * 2));
#pragma unroll
    for (int j = 0; j < FN2; ++j) {
      const int u = T1 + kt * FN2 + j;
      const bf16x8(&w)[3][2] = ring[u % PD];
#pragma unroll
      for (int s = 0; s < 2; ++s) {
        acc2[j] = fm_mfma32_bf16(a[1][s], w[1][s], acc2[j]);
        acc2[j] = fm_mfma32_bf16(a[2][s], w[0][s], acc2[j]);
        acc2[j] = fm_mfma32_bf16(a[1][s], w[0][s], acc2[j]);
        acc2[j] = fm_mfma32_bf16(a[0][s], w[2][s], acc2[j]);
        acc2[j] = fm_mfma32_bf16(a[0][s], w[1][s], acc2[j]);
        acc2[j] = fm_mfma32_bf16(a[0][s], w[0][s], acc2[j]);
      }
      if (u + PD < T) load_unit(u + PD, ring[u % PD]);
      __builtin_amdgcn_sched_barrier(0);
    }
  }
  if constexpr (WAVE_OUT) {
    // Output rows into this wave's [32][68] tile (over the consumed planes),
    // then lane (r, half hh) forms w3[j] . y[r] over 32 channels and the
    // halves are summed: D[b][t] = {d0, d1, d2, 0}.
    __syncthreads();
    float* E = reinterpret_cast<float*>(smem) + wave * 32 * 68;
#pragma unroll
    for (int j = 0; j < FN2; ++j) {
      const float bias = b2[j * 32 + lcol];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = __fadd_rn(rv[j][r], __fadd_rn(acc2[j][r], bias));
        if (elu_out) v = act(v);
        E[fm_mfma32_row(r, lane) * 68 + j * 32 + lcol] = v;
      }
    }
    wave_lds_fence();
    const int r = lane & 31, hh = lane >> 5;
    float d[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 32; c += 4) {
      const floatx4 v = *reinterpret_cast<const floatx4*>(E + r * 68 + 32 * hh + c);
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const floatx4 wj = *reinterpret_cast<const floatx4*>(w0 + j * 64 + 32 * hh + c);
        d[j] = fmaf(wj[0], v[0], d[j]);
        d[j] = fmaf(wj[1], v[1], d[j]);
        d[j] = fmaf(wj[2], v[2], d[j]);
        d[j] = fmaf(wj[3], v[3], d[j]);
      }
    }
    floatx4 o;
#pragma unroll
    for (int j = 0; j < 3; ++j) o[j] = __fadd_rn(d[j], __shfl_xor(d[j], 32, 64));
    o[3] = 0.0f;
    const int t = t0 + wr * 32 + r;
    if (hh == 0 && t < L) *reinterpret_cast<floatx4*>(y + (b * L + t) * 4) = o;
    return;
  }
#pragma unroll
  for (int j = 0; j < FN2; ++j) {
    const int n = wc * 64 + j * 32 + lcol;
    const float bias = b2[n];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int t = t0 + wr * 32 + fm_mfma32_row(r, lane);
      float v = __fadd_rn(rv[j][r], __fadd_rn(acc2[j][r], bias));
      if (elu_out) v = act(v);
      if (fast) {
        fm_buf_store1(v, ry, vrow, row_off(r, j));
      } else if (t < L) {
        yb[(long)t * C + n] = v;
      }
    }
  }
}

}  // namespace

// The bf16x6 planes stored after a packed weight W^T [rows][cols].
static const __bf16* planes_after(const float* w, int rows, int cols) {
  return reinterpret_cast<const __bf16*>(w + (long)rows * cols);
}

extern "C" {

// Channel widths with a fused kernel; others run as two fm_conv1d calls.
int fm_resblock_supported(int channels) {
  return channels == 64 || channels == 128 || channels == 256;
}

int fm_resblock(const float* x, int batch, int length, int channels, const float* w1_packed,
                const float* b1, const float* w2_packed, const float* b2, int elu_out, float* y,
                hipStream_t stream) {
  if (!x || !w1_packed || !b1 || !w2_packed || !b2 || !y || batch < 0 || length < 0)
    return FM_BAD_ARGUMENT;
  if (!fm_resblock_supported(channels)) return FM_UNSUPPORTED;
  if (x == y) return FM_BAD_ARGUMENT;  // the halo rows of other blocks must stay intact
  if (batch == 0 || length == 0) return FM_OK;
  const int elu = (elu_out & ~(FM_WEIGHTS_X6 | FM_ACT_EXP)) != 0;
  const bool x6 = elu_out & FM_WEIGHTS_X6, fa = elu_out & FM_ACT_EXP;
  if (x6) {
    // Split planes follow each packed weight (fm_split_weights).
    const __bf16* w1x = planes_after(w1_packed, channels / 2, 3 * channels);
    const __bf16* w2x = planes_after(w2_packed, channels, channels / 2);
#define FM_RB(C_, BM_, WM_, FA_)                                                                    \
  hipLaunchKernelGGL((resblock_x6_kernel<C_, BM_, WM_, 2, false, false, FA_>), dim3((length + BM_ - 1) / BM_, batch), \
                     dim3(NT), 0, stream, x, length, w1x, b1, w2x, b2, elu, y, nullptr, nullptr)
    if (channels == 64) {
      if (fa) FM_RB(64, 128, 4, true); else FM_RB(64, 128, 4, false);
    } else if (channels == 128) {
      if (fa) FM_RB(128, 64, 2, true); else FM_RB(128, 64, 2, false);
    } else {
      if (fa) FM_RB(256, 32, 1, true); else FM_RB(256, 32, 1, false);
    }
#undef FM_RB
  } else if (channels == 64) {
    // Persistent: one 12-wave block per CU (LDS-bound), waves stride over 32-row tiles.
    const long tiles = (long)batch * ((length + 31) / 32);
    const int blocks = (int)std::min<long>((tiles + R64_WAVES - 1) / R64_WAVES, 256);
    hipLaunchKernelGGL((resblock64_kernel<false, false>), dim3(blocks), dim3(64 * R64_WAVES), 0, stream, x,
                       batch, length, w1_packed, b1, w2_packed, b2, elu, y, nullptr, nullptr);
  } else if (channels == 128) {
    hipLaunchKernelGGL((resblock_direct_kernel<128, 64, 2, 3>), dim3((length + 63) / 64, batch), dim3(NT),
                       0, stream, x, length, w1_packed, b1, w2_packed, b2, elu, y);
  } else {
    hipLaunchKernelGGL((resblock_direct_kernel<256, 32, 1, 3>), dim3((length + 31) / 32, batch), dim3(NT),
                       0, stream, x, length, w1_packed, b1, w2_packed, b2, elu, y);
  }
  return (int)hipGetLastError();
}

// The encoder's first conv (1 -> 64 channels, kernel 7, causal) fused into
// the residual block that follows it: y = block(conv(wav)).
int fm_conv_resblock64(const float* wav, int batch, int length, const float* w0_packed,
                       const float* b0, const float* w1_packed, const float* b1,
                       const float* w2_packed, const float* b2, int elu_out, float* y,
                       hipStream_t stream) {
  if (!wav || !w0_packed || !b0 || !w1_packed || !b1 || !w2_packed || !b2 || !y || batch < 0 ||
      length < 0)
    return FM_BAD_ARGUMENT;
  if (batch == 0 || length == 0) return FM_OK;
  const int elu = (elu_out & ~(FM_WEIGHTS_X6 | FM_ACT_EXP)) != 0;
  if (elu_out & FM_WEIGHTS_X6) {
    if (elu_out & FM_ACT_EXP)
      hipLaunchKernelGGL((resblock_x6_kernel<64, 128, 4, 2, true, false, true>), dim3((length + 127) / 128, batch),
                         dim3(NT), 0, stream, wav, length, planes_after(w1_packed, 32, 192), b1,
                         planes_after(w2_packed, 64, 32), b2, elu, y, w0_packed, b0);
    else
      hipLaunchKernelGGL((resblock_x6_kernel<64, 128, 4, 2, true, false>), dim3((length + 127) / 128, batch),
                         dim3(NT), 0, stream, wav, length, planes_after(w1_packed, 32, 192), b1,
                         planes_after(w2_packed, 64, 32), b2, elu, y, w0_packed, b0);
    return (int)hipGetLastError();
  }
  const long tiles = (long)batch * ((length + 31) / 32);
  const int blocks = (int)std::min<long>((tiles + R64_WAVES - 1) / R64_WAVES, 256);
  hipLaunchKernelGGL((resblock64_kernel<true, false>), dim3(blocks), dim3(64 * R64_WAVES), 0, stream, wav,
                     batch, length, w1_packed, b1, w2_packed, b2, elu, y, w0_packed, b0);
  return (int)hipGetLastError();
}

// The decoder's last 64-channel residual block fused with the waveform conv
// after it (64 -> 1 channel, kernel 3, causal): out = conv(block(x)) cropped
// to y_len rows.  workspace: fm_resblock64_conv_workspace_bytes.
size_t fm_resblock64_conv_workspace_bytes(int batch, int length) {
  return (size_t)batch * length * 4 * sizeof(float);
}

int fm_resblock64_conv(const float* x, int batch, int length, const float* w1_packed,
                       const float* b1, const float* w2_packed, const float* b2, int elu_mid,
                       const float* w3_packed, const float* b3, int y_len, float* out,
                       float* workspace, size_t workspace_bytes, hipStream_t stream) {
  if (!x || !w1_packed || !b1 || !w2_packed || !b2 || !w3_packed || !out || batch < 0 ||
      length < 0 || y_len < 0 || y_len > length)
    return FM_BAD_ARGUMENT;
  if (batch == 0 || y_len == 0) return FM_OK;
  if (!workspace || workspace_bytes < fm_resblock64_conv_workspace_bytes(batch, length))
    return FM_WORKSPACE_TOO_SMALL;
  const int elu = (elu_mid & ~(FM_WEIGHTS_X6 | FM_ACT_EXP)) != 0;
  if (elu_mid & FM_WEIGHTS_X6) {
    if (elu_mid & FM_ACT_EXP)
      hipLaunchKernelGGL((resblock_x6_kernel<64, 128, 4, 2, false, true, true>), dim3((length + 127) / 128, batch),
                         dim3(NT), 0, stream, x, length, planes_after(w1_packed, 32, 192), b1,
                         planes_after(w2_packed, 64, 32), b2, elu, workspace, w3_packed, nullptr);
    else
      hipLaunchKernelGGL((resblock_x6_kernel<64, 128, 4, 2, false, true>), dim3((length + 127) / 128, batch),
                         dim3(NT), 0, stream, x, length, planes_after(w1_packed, 32, 192), b1,
                         planes_after(w2_packed, 64, 32), b2, elu, workspace, w3_packed, nullptr);
  } else {
    const long tiles = (long)batch * ((length + 31) / 32);
    const int blocks = (int)std::min<long>((tiles + R64_WAVES - 1) / R64_WAVES, 256);
    hipLaunchKernelGGL((resblock64_kernel<false, true>), dim3(blocks), dim3(64 * R64_WAVES), 0, stream,
                       x, batch, length, w1_packed, b1, w2_packed, b2, elu, workspace, w3_packed,
                       nullptr);
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  hipLaunchKernelGGL(conv3_finish_kernel, dim3((y_len + 255) / 256, batch), dim3(256), 0, stream,
                     workspace, length, y_len, b3, out);
  return (int)hipGetLastError();
}

}  // extern "C"
