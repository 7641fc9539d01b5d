// Fused SEANet residual block (kadirnar/fast-mimi src/fast_mimi/model.py:947-971):
//
//   y = ELU?( x + conv1x1( ELU( conv_k3( ELU(x) ) + b1 ) ) + b2 )
//
// on channels-last x [batch, L, C] with causal (left) zero padding of 2 and
// hidden width C/2.  One block owns BM consecutive positions of one batch
// item.  ELU(x) for rows t0-2 .. t0+BM-1 (the causal halo included) is staged
// in LDS once; the k3 convolution reads its three taps as row-shifted views
// of that tile, so the input is read from HBM once instead of once per tap.
// The hidden activations never leave LDS; the 1x1 convolution adds the raw
// residual (read once, coalesced) and the block's trailing ELU in its
// epilogue.  Both GEMMs run on FP32 MFMA with the k-permuted 16-byte fragment
// reads of the main GEMM engine (k-slot of lane half h at step 4q+e carries
// k = 16h + 4q + e).  Weights stream through a double-buffered LDS tile fed
// from a 3-deep register prefetch ring: W1^T [C/2][3C] (k = tap*C + c_in, the
// packed conv layout) then W2^T [C][C/2].

#include "fm_common.h"

namespace {

constexpr int NT = 256;

// WBK: weight k-tile (16 keeps the LDS footprint low enough for two blocks
// per CU at C = 128, so a second block's MFMAs cover one block's barriers).
template <int C, int BM, int WM1, int WN1, int WM2, int WN2, int WBK>
__global__ __launch_bounds__(NT) void resblock_kernel(const float* __restrict__ x, int L,
                                                      const float* __restrict__ w1,
                                                      const float* __restrict__ b1,
                                                      const float* __restrict__ w2,
                                                      const float* __restrict__ b2, int elu_out,
                                                      float* __restrict__ y) {
  constexpr int PW = WBK + 4;       // weight tile pitch
  constexpr int HK = WBK / 2;       // k per MFMA lane half within a weight tile
  constexpr int HC = C / 2;
  constexpr int K1 = 3 * C;
  constexpr int T1 = K1 / WBK, T2 = HC / WBK, T = T1 + T2;
  constexpr int PX = C + 4, PH = HC + 4;
  constexpr int FM1 = BM / WM1 / 32, FN1 = HC / WN1 / 32;
  constexpr int FM2 = BM / WM2 / 32, FN2 = C / WN2 / 32;
  constexpr int WROWS = C;                      // max rows of a weight tile
  constexpr int WPT = (WROWS * WBK / 4) / NT;   // float4 per thread (W2 tiles)
  static_assert(WM1 * WN1 == 4 && WM2 * WN2 == 4, "four waves");
  static_assert(FM1 >= 1 && FN1 >= 1 && FM2 >= 1 && FN2 >= 1, "32x32 wave tiles");
  static_assert(HC % WBK == 0 && WPT >= 1, "shapes");

  __shared__ __attribute__((aligned(16))) float Xe[(BM + 2) * PX];
  __shared__ __attribute__((aligned(16))) float Hs[BM * PH];
  __shared__ __attribute__((aligned(16))) float Ws[2][WROWS * PW];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  const long b = blockIdx.y;
  const int t0 = blockIdx.x * BM;
  const float* xb = x + b * (long)L * C;

  // Stage ELU(x) rows t0-2 .. t0+BM-1; loads batched ahead of the stores.
  {
    constexpr int CH = (BM + 2) * C / 4;
    constexpr int U = (CH + NT - 1) / NT;
    floatx4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = tid + u * NT;
      const int r = c / (C / 4), k = (c % (C / 4)) * 4;
      const int t = t0 - 2 + r;
      v[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (c < CH && t >= 0 && t < L) v[u] = *reinterpret_cast<const floatx4*>(xb + (long)t * C + k);
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int c = tid + u * NT;
      if (c >= CH) continue;
      const int r = c / (C / 4), k = (c % (C / 4)) * 4;
      *reinterpret_cast<floatx4*>(&Xe[r * PX + k]) =
          floatx4{fm_elu(v[u].x), fm_elu(v[u].y), fm_elu(v[u].z), fm_elu(v[u].w)};
    }
  }

  // Weight tile w: rows of W1^T (w < T1) or W2^T, k columns [k0, k0 + 32).
  // Tiles are fetched PD iterations ahead into a ring of register sets, so a
  // tile's global-load latency overlaps PD iterations of MFMA work.
  constexpr int PD = 3;
  floatx4 rw[PD][WPT];
  auto load_w = [&](int w, floatx4 (&dst)[WPT]) {
    const bool first = w < T1;
    const int rows = first ? HC : C;
    const int ld = first ? K1 : HC;
    const float* src = first ? w1 : w2;
    const int k0 = (first ? w : w - T1) * WBK;
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
      const int c = tid + u * NT;
      const int r = c / (WBK / 4), k = (c % (WBK / 4)) * 4;
      dst[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (w < T && r < rows) dst[u] = *reinterpret_cast<const floatx4*>(src + (long)r * ld + k0 + k);
    }
  };
  auto store_w = [&](int stage, const floatx4 (&srcv)[WPT]) {
#pragma unroll
    for (int u = 0; u < WPT; ++u) {
      const int c = tid + u * NT;
      const int r = c / (WBK / 4), k = (c % (WBK / 4)) * 4;
      *reinterpret_cast<floatx4*>(&Ws[stage][r * PW + k]) = srcv[u];
    }
  };

  floatx16 acc1[FM1][FN1];
  floatx16 acc2[FM2][FN2];
#pragma unroll
  for (int i = 0; i < FM1; ++i)
#pragma unroll
    for (int j = 0; j < FN1; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc1[i][j][r] = 0.0f;
#pragma unroll
  for (int i = 0; i < FM2; ++i)
#pragma unroll
    for (int j = 0; j < FN2; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc2[i][j][r] = 0.0f;

  const int wm1 = (wave / WN1) * (BM / WM1), wn1 = (wave % WN1) * (HC / WN1);
  const int wm2 = (wave / WN2) * (BM / WM2), wn2 = (wave % WN2) * (C / WN2);

#pragma unroll
  for (int d = 0; d < PD; ++d) load_w(d, rw[d]);
  store_w(0, rw[0]);
  __syncthreads();
#pragma unroll
  for (int w = 0; w < T; ++w) {
    const int cur = w & 1;
    if (w + PD < T) load_w(w + PD, rw[w % PD]);  // set w % PD was stored to LDS already
    const float* Wc = Ws[cur];
    if (w < T1) {
      const int kk0 = w * WBK;
      const int tap = kk0 / C, ci0 = kk0 % C;
#pragma unroll
      for (int s4 = 0; s4 < WBK / 8; ++s4) {
        floatx4 a[FM1], bb[FN1];
#pragma unroll
        for (int i = 0; i < FM1; ++i)
          a[i] = *reinterpret_cast<const floatx4*>(&Xe[(wm1 + i * 32 + lcol + tap) * PX + ci0 + h * HK + s4 * 4]);
#pragma unroll
        for (int j = 0; j < FN1; ++j)
          bb[j] = *reinterpret_cast<const floatx4*>(&Wc[(wn1 + j * 32 + lcol) * PW + h * HK + s4 * 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < FM1; ++i)
#pragma unroll
            for (int j = 0; j < FN1; ++j) acc1[i][j] = fm_mfma32(a[i][e], bb[j][e], acc1[i][j]);
      }
      if (w == T1 - 1) {
        // Hidden activations: ELU(conv_k3 + b1) into LDS.
#pragma unroll
        for (int j = 0; j < FN1; ++j) {
          const int n = wn1 + j * 32 + lcol;
          const float bias = b1[n];
#pragma unroll
          for (int i = 0; i < FM1; ++i)
#pragma unroll
            for (int r = 0; r < 16; ++r)
              Hs[(wm1 + i * 32 + fm_mfma32_row(r, lane)) * PH + n] = fm_elu(__fadd_rn(acc1[i][j][r], bias));
        }
      }
    } else {
      const int kk0 = (w - T1) * WBK;
#pragma unroll
      for (int s4 = 0; s4 < WBK / 8; ++s4) {
        floatx4 a[FM2], bb[FN2];
#pragma unroll
        for (int i = 0; i < FM2; ++i)
          a[i] = *reinterpret_cast<const floatx4*>(&Hs[(wm2 + i * 32 + lcol) * PH + kk0 + h * HK + s4 * 4]);
#pragma unroll
        for (int j = 0; j < FN2; ++j)
          bb[j] = *reinterpret_cast<const floatx4*>(&Wc[(wn2 + j * 32 + lcol) * PW + h * HK + s4 * 4]);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < FM2; ++i)
#pragma unroll
            for (int j = 0; j < FN2; ++j) acc2[i][j] = fm_mfma32(a[i][e], bb[j][e], acc2[i][j]);
      }
    }
    if (w + 1 < T) store_w(cur ^ 1, rw[(w + 1) % PD]);
    __syncthreads();
  }

  // y = ELU?(x + (conv1x1 + b2)), rows t < L.  Residual loads are all issued
  // before any store so they overlap.
  float* yb = y + b * (long)L * C;
  float rv[FN2][FM2][16];
#pragma unroll
  for (int j = 0; j < FN2; ++j)
#pragma unroll
    for (int i = 0; i < FM2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = min(t0 + wm2 + i * 32 + fm_mfma32_row(r, lane), L - 1);
        rv[j][i][r] = xb[(long)t * C + wn2 + j * 32 + lcol];
      }
#pragma unroll
  for (int j = 0; j < FN2; ++j) {
    const int n = wn2 + j * 32 + lcol;
    const float bias = b2[n];
#pragma unroll
    for (int i = 0; i < FM2; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int t = t0 + wm2 + i * 32 + fm_mfma32_row(r, lane);
        float v = __fadd_rn(rv[j][i][r], __fadd_rn(acc2[i][j][r], bias));
        if (elu_out) v = fm_elu(v);
        if (t < L) yb[(long)t * C + n] = v;
      }
  }
}


// ---------------------------------------------------------------------------
// C = 64 residual block as a persistent kernel.  The block's weights are
// staged once in LDS as MFMA B-fragment rows (W1^T [32][192], W2^T [64][32]),
// shared by the 8 waves.  Each wave then takes 32-row tiles in a grid-stride
// loop with no block-level barrier: stage ELU(x) rows t0-2 .. t0+31 in its own
// LDS slot, issue the residual rows of this tile and the input rows of its
// next tile (both land during the MFMAs), k3 conv (96 MFMAs in two chains,
// taps as row-shifted views), hidden = ELU(acc + b1) into LDS, 1x1 conv (32
// MFMAs), then the output tile goes back through LDS so the epilogue (bias,
// raw residual, ELU) runs on float4 runs.  Two waves per SIMD overlap one
// tile's memory and ELU work with the other's MFMAs.  MFMA k-slots: lane half
// h at step 4q+e carries k = 96h + 4q + e (k3 conv, k = tap*64 + c_in) or
// 16h + 4q + e (1x1 conv).
constexpr int R64_WAVES = 8;
constexpr int R64_PE = 68;   // pitch of the ELU(x) / output tile rows
constexpr int R64_PH = 36;   // pitch of the hidden tile rows
constexpr int R64_SLOT = 34 * R64_PE + 32 * R64_PH;
constexpr int R64_P1 = 196;  // W1^T row pitch (4 mod 32: conflict-free 16-byte reads)
constexpr int R64_P2 = 36;   // W2^T row pitch

__global__ __launch_bounds__(64 * R64_WAVES) void resblock64_kernel(
    const float* __restrict__ x, int batch, int L, const float* __restrict__ w1,
    const float* __restrict__ b1, const float* __restrict__ w2, const float* __restrict__ b2,
    int elu_out, float* __restrict__ y) {
  constexpr int C = 64, HC = 32;
  __shared__ __attribute__((aligned(16))) float smem[R64_WAVES * R64_SLOT + 32 * R64_P1 + 64 * R64_P2];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  float* E = smem + wave * R64_SLOT;   // [34][68] ELU(x); later the [32][68] output tile
  float* H = E + 34 * R64_PE;          // [32][36] hidden
  float* W1s = smem + R64_WAVES * R64_SLOT;
  float* W2s = W1s + 32 * R64_P1;

  for (int i = threadIdx.x; i < 32 * 48; i += 64 * R64_WAVES) {
    const int r = i / 48, c4 = (i % 48) * 4;
    *reinterpret_cast<floatx4*>(W1s + r * R64_P1 + c4) = *reinterpret_cast<const floatx4*>(w1 + r * 192 + c4);
  }
  for (int i = threadIdx.x; i < 64 * 8; i += 64 * R64_WAVES) {
    const int r = i / 8, c4 = (i % 8) * 4;
    *reinterpret_cast<floatx4*>(W2s + r * R64_P2 + c4) = *reinterpret_cast<const floatx4*>(w2 + r * HC + c4);
  }
  const float bias1 = b1[lcol];
  __syncthreads();

  const int tpb = (L + 31) / 32;
  const long tiles = (long)batch * tpb;
  const long stride = (long)gridDim.x * R64_WAVES;
  long tile = (long)blockIdx.x * R64_WAVES + wave;

  // x rows t0-2 .. t0+31 of a tile: 544 float4 chunks, 9 per lane (chunk c = lane + 64u).
  floatx4 xv[9];
  unsigned xok = 0;
  auto load_x = [&](long tl) {
    const int b = (int)(tl / tpb), t0 = (int)(tl % tpb) * 32;
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
  if (tile < tiles) load_x(tile);
  for (; tile < tiles; tile += stride) {
    const int b = (int)(tile / tpb), t0 = (int)(tile % tpb) * 32;
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
    floatx4 rv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) {
      const int c = lane + 64 * u;
      rv[u] = *reinterpret_cast<const floatx4*>(xb + (long)min(t0 + c / 16, L - 1) * C + (c % 16) * 4);
    }
    if (tile + stride < tiles) load_x(tile + stride);
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
    // Output tile through LDS (the ELU(x) rows are no longer read).
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
      if (t0 + r < L) *reinterpret_cast<floatx4*>(yb + (long)(t0 + r) * C + c4) = v;
    }
    wave_lds_fence();  // the slot is rewritten by the next tile
  }
}

}  // namespace

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
#define FM_RB(C, BM, A, B_, C2, D, KB)                                                              \
  hipLaunchKernelGGL((resblock_kernel<C, BM, A, B_, C2, D, KB>), dim3((length + BM - 1) / BM, batch), \
                     dim3(NT), 0, stream, x, length, w1_packed, b1, w2_packed, b2, elu_out, y)
  if (channels == 64) {
    // Persistent: one 8-wave block per CU (LDS-bound), waves stride over 32-row tiles.
    const long tiles = (long)batch * ((length + 31) / 32);
    const int blocks = (int)std::min<long>((tiles + R64_WAVES - 1) / R64_WAVES, 256);
    hipLaunchKernelGGL(resblock64_kernel, dim3(blocks), dim3(64 * R64_WAVES), 0, stream, x, batch,
                       length, w1_packed, b1, w2_packed, b2, elu_out, y);
    return (int)hipGetLastError();
  }
  switch (channels) {
    case 64: FM_RB(64, 128, 4, 1, 4, 1, 32); break;
    case 128: FM_RB(128, 64, 2, 2, 2, 2, 16); break;
    default: FM_RB(256, 32, 1, 4, 1, 4, 32); break;
  }
#undef FM_RB
  return (int)hipGetLastError();
}

}  // extern "C"
