// Few-row convolutions with long K: the 12.5 / 25 Hz end of the SEANet stacks
// at B x T <= 512 output rows (the encoder's last conv 1024 -> 512 k3, the
// bottleneck's replicate-padded downsample 512 -> 512 k4 s2, the decoder's
// first conv 512 -> 1024 k7).  The tiled GEMM engine has a few dozen tiles
// there and splits K across blocks with a second reduce launch; this kernel
// instead gives every 16 output rows x BN columns (32, or 64 where 32-column
// blocks would not all be resident at once) one block of 8 waves that split
// K, as the transformer's row-block projections do, and sums the 8 partial
// tiles through LDS in wave order.
//
// Weights are the conv's W^T [N][K] (k = tap * C_in + c) in the fragment
// order of fm_pack_row_weights: the float4 at ((nt * (K/64) + kp) * 4 + t) *
// 64 + lane holds W^T[16 nt + lane % 16][64 kp + 16 (lane / 16) + 4 t .. + 3],
// so a wave's B fragment of a 64-deep piece is one 1 KB run.  The A fragment
// of lane (row li = lane % 16, group g = lane / 16) in a piece is 16
// consecutive floats of one input position: C_in is a multiple of 64, so a
// 64-deep piece never crosses a tap, and the position is the output row's
// window start plus the piece's tap (zero outside the signal, or clamped to
// its ends with replicate padding).  Both operands of the next piece are
// loaded into registers while the current one runs on v_mfma_f32_16x16x4f32.

#include "fm_common.h"

namespace {

__device__ __attribute__((aligned(16))) float g_zero_row[16];

struct RowConvArgs {
  const float* x;    // [batch][L][C_in]
  const float* w;    // fragment-packed W^T [N][K]
  const float* bias; // [bias_len], or null
  const float* res;  // [batch][rows_per_batch][N] with FM_EPI_RES_ADD, else null
  float* y;          // [batch][rows_per_batch][N]
  int L, c_in, stride, pad_l, replicate, rows_per_batch, rows, N, bias_len, flags;
};

template <int K, int BN, bool X6, int MT>
__global__ __launch_bounds__(512) void row16_conv_kernel(RowConvArgs p) {
  // MT 16-row MFMA tiles per block (bf16x6 only): each weight fragment a wave
  // loads serves all of them, so the weights cross L2 once per 16 * MT rows.
  constexpr int NWV = 8, BM = 16 * MT, KW = K / NWV, NP = KW / 64, NT = BN / 16;
  constexpr int PR = BN + 4, OPT = BM * BN / 512;
  static_assert((X6 ? KW % 32 : KW % 64) == 0 && OPT >= 1 && (X6 || MT == 1), "tile shape");
  __shared__ __attribute__((aligned(16))) float red[NWV * BM * PR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const long m0 = (long)blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int kw0 = wave * KW;

  // This lane's output rows li + 16 mt (clamped: rows past the end load a
  // valid row and are not stored) and their window starts.
  int p0[MT];
  const float* xb[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) {
    const long mr = min(m0 + 16 * mt + li, (long)p.rows - 1);
    const int b = (int)(mr / p.rows_per_batch);
    const int t = (int)(mr - (long)b * p.rows_per_batch);
    p0[mt] = t * p.stride - p.pad_l;
    xb[mt] = p.x + (long)b * p.L * p.c_in;
  }
  // Input run of row tile mt for the k-range starting at k (wave-uniform; the
  // range lies inside one tap).
  auto a_src = [&](int mt, int k, int lane_off) -> const float* {
    const int tap = k / p.c_in;
    int pos = p0[mt] + tap;
    if (p.replicate) pos = min(max(pos, 0), p.L - 1);
    else if ((unsigned)pos >= (unsigned)p.L) return g_zero_row;
    return xb[mt] + (long)pos * p.c_in + (k - tap * p.c_in) + lane_off;
  };
  const bool elu_in = p.flags & FM_ELU_IN;
  floatx4 acc[MT][NT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j) acc[mt][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  if constexpr (X6) {
    // bf16x6: W^T's planes [3][K/16][N][16] after the FP32 weight; 32-deep k
    // steps on v_mfma_f32_16x16x32_bf16, lane group g covering k = 8g .. 8g+7
    // of A and B.  Units (step, plane) stream through a ring of R weight
    // fragments; A runs RA - 1 steps ahead and is split as it is used.  The
    // unit loop is unrolled by CHU units so every ring index is static.
    constexpr int KS = KW / 32, NU = 3 * KS;
    constexpr int RA = MT == 1 ? (KS % 4 == 0 ? 4 : KS % 2 == 0 ? 2 : 1) : (KS % 2 == 0 ? 2 : 1);
    constexpr int CHU = 3 * RA, R = CHU >= 6 && NT == 2 && MT == 1 ? 6 : 3;
    static_assert(KW % 32 == 0 && KS % RA == 0 && CHU % R == 0, "whole 32-deep steps per wave");
    const __bf16* w3 = reinterpret_cast<const __bf16*>(p.w + (long)p.N * K);
    const long PL = (long)p.N * K;
    const __bf16* wb3 = w3 + ((long)((kw0 >> 4) + (g >> 1)) * p.N + n0 + li) * 16 + 8 * (g & 1);
    bf16x8 bu[R][NT];
    floatx4 a3[RA][MT][2];
    auto load_unit = [&](int buf, int u) {
      if (u >= NU) return;
      const int st = u / 3, pl = u - 3 * st;
#pragma unroll
      for (int j = 0; j < NT; ++j)
        bu[buf][j] = *reinterpret_cast<const bf16x8*>(wb3 + pl * PL + (long)st * 2 * p.N * 16 + j * 256);
    };
    auto load_a3 = [&](int buf, int st) {
      if (st >= KS) return;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const float* src = a_src(mt, kw0 + 32 * st, 8 * g);
        a3[buf][mt][0] = *reinterpret_cast<const floatx4*>(src);
        a3[buf][mt][1] = *reinterpret_cast<const floatx4*>(src + 4);
      }
    };
#pragma unroll
    for (int u = 0; u + 1 < R; ++u) load_unit(u, u);
#pragma unroll
    for (int st = 0; st + 1 < RA; ++st) load_a3(st, st);
    __builtin_amdgcn_sched_barrier(0);
    bf16x8 p0v[MT], p1v[MT], p2v[MT];
    for (int u0 = 0; u0 < NU; u0 += CHU) {
#pragma unroll
      for (int i = 0; i < CHU; ++i) {
        const int u = u0 + i;
        const int pl = i % 3, c = i % R;
        load_unit((i + R - 1) % R, u + R - 1);
        if (pl == 0) {
          const int sa = i / 3;  // u0 / 3 is a multiple of RA
          load_a3((sa + RA - 1) % RA, u / 3 + RA - 1);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) {
            floatx4 v0 = a3[sa % RA][mt][0], v1 = a3[sa % RA][mt][1];
            if (elu_in) {
#pragma unroll
              for (int e = 0; e < 4; ++e) v0[e] = fm_elu(v0[e]), v1[e] = fm_elu(v1[e]);
            }
            bf16x4 l0, l1, l2, h0, h1, h2;
            split3(v0, l0, l1, l2);
            split3(v1, h0, h1, h2);
            p0v[mt] = __builtin_shufflevector(l0, h0, 0, 1, 2, 3, 4, 5, 6, 7);
            p1v[mt] = __builtin_shufflevector(l1, h1, 0, 1, 2, 3, 4, 5, 6, 7);
            p2v[mt] = __builtin_shufflevector(l2, h2, 0, 1, 2, 3, 4, 5, 6, 7);
          }
        }
        __builtin_amdgcn_sched_barrier(0);
        // Plane 0 of W meets all three A pieces, plane 1 the first two,
        // plane 2 the first: the six terms of order <= 2.
#pragma unroll
        for (int mt = 0; mt < MT; ++mt) {
          if (pl == 0) {
#pragma unroll
            for (int j = 0; j < NT; ++j)
              acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p2v[mt], bu[c][j], acc[mt][j], 0, 0, 0);
#pragma unroll
            for (int j = 0; j < NT; ++j)
              acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p1v[mt], bu[c][j], acc[mt][j], 0, 0, 0);
          } else if (pl == 1) {
#pragma unroll
            for (int j = 0; j < NT; ++j)
              acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p1v[mt], bu[c][j], acc[mt][j], 0, 0, 0);
          }
#pragma unroll
          for (int j = 0; j < NT; ++j)
            acc[mt][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(p0v[mt], bu[c][j], acc[mt][j], 0, 0, 0);
        }
      }
    }
  } else {
    const long tstride = (long)(K / 64) * 4 * 64 * 4;  // floats between 16-column tiles
    const float* wb = p.w + ((((long)(n0 / 16) * (K / 64) + kw0 / 64) * 4) * 64 + lane) * 4;
    floatx4 a[2][4], bw[2][NT][4];
    auto load = [&](int buf, int piece) {
#pragma unroll
      for (int j = 0; j < NT; ++j)
#pragma unroll
        for (int q = 0; q < 4; ++q)
          bw[buf][j][q] = *reinterpret_cast<const floatx4*>(wb + j * tstride + piece * 1024 + q * 256);
      const float* src = a_src(0, kw0 + 64 * piece, 16 * g);
#pragma unroll
      for (int q = 0; q < 4; ++q) a[buf][q] = *reinterpret_cast<const floatx4*>(src + 4 * q);
    };
    load(0, 0);
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int pc = 0; pc < NP; ++pc) {
      const int c = pc & 1;
      if (pc + 1 < NP) load(c ^ 1, pc + 1);
      __builtin_amdgcn_sched_barrier(0);
      if (elu_in) {
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int e = 0; e < 4; ++e) a[c][q][e] = fm_elu(a[c][q][e]);
      }
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int j = 0; j < NT; ++j)
            acc[0][j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c][q][e], bw[c][j][q][e], acc[0][j], 0, 0, 0);
    }
  }

  // The 8 partial tiles summed in wave order, then bias, residual and the
  // output ELU.
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(wave * BM + 16 * mt + 4 * g + r) * PR + 16 * j + li] = acc[mt][j][r];
  __syncthreads();
  const int er = tid / (BN / OPT), ec = (tid % (BN / OPT)) * OPT;
  const long m = m0 + er;
  if (m >= p.rows) return;
  float out[OPT];
#pragma unroll
  for (int c = 0; c < OPT; ++c) {
    float v = red[er * PR + ec + c];
#pragma unroll
    for (int q = 1; q < NWV; ++q) v = __fadd_rn(v, red[(q * BM + er) * PR + ec + c]);
    if (p.bias) v = __fadd_rn(v, p.bias[(n0 + ec + c) % p.bias_len]);
    if (p.flags & FM_EPI_RES_ADD) v = __fadd_rn(p.res[m * p.N + n0 + ec + c], v);
    if (p.flags & FM_EPI_ELU) v = fm_elu(v);
    out[c] = v;
  }
  float* dst = p.y + m * p.N + n0 + ec;
#pragma unroll
  for (int c = 0; c < OPT; ++c) dst[c] = out[c];
}

}  // namespace

extern "C" {

int fm_conv1d_rows_supported(int in_channels, int out_channels, int kernel, int flags) {
  const int K = in_channels * kernel;
  if (out_channels % 32) return 0;
  if (flags & FM_WEIGHTS_X6)
    return in_channels % 32 == 0 && (K == 256 || K == 1536 || K == 2048 || K == 3072 || K == 3584);
  return in_channels % 64 == 0 && (K == 1536 || K == 2048 || K == 3072 || K == 3584);
}

int fm_conv1d_rows(const float* x, int batch, int length, int in_channels, const float* weight,
                   const float* bias, int bias_len, int out_channels, int kernel, int stride,
                   int pad_mode, int flags, const float* residual, float* y, hipStream_t stream) {
  if (!x || !weight || !y || batch < 0 || length < 0 || kernel <= 0 || stride <= 0 ||
      kernel < stride || (pad_mode != 0 && pad_mode != 1) || (bias && bias_len <= 0) ||
      (flags & FM_EPI_RES_ADD && !residual))
    return FM_BAD_ARGUMENT;
  if (flags & ~(FM_ELU_IN | FM_EPI_ELU | FM_EPI_RES_ADD | FM_WEIGHTS_X6)) return FM_UNSUPPORTED;
  if (!fm_conv1d_rows_supported(in_channels, out_channels, kernel, flags)) return FM_UNSUPPORTED;
  const int rows_per_batch = (length + stride - 1) / stride;
  const long rows = (long)batch * rows_per_batch;
  if (rows == 0) return FM_OK;
  if (length == 0) return FM_BAD_ARGUMENT;
  if ((rows + 15) / 16 > 65535) return FM_UNSUPPORTED;
  RowConvArgs p{x, weight, bias, flags & FM_EPI_RES_ADD ? residual : nullptr, y, length, in_channels,
                stride, kernel - stride, pad_mode, rows_per_batch, (int)rows, out_channels,
                bias ? bias_len : 1, flags};
  const unsigned row_blocks = (unsigned)((rows + 15) / 16);
  const dim3 grid(out_channels / 32, row_blocks);
  const int K = in_channels * kernel;
#define FM_ROWCONV(KK, X6) hipLaunchKernelGGL((row16_conv_kernel<KK, 32, X6, 1>), grid, dim3(512), 0, stream, p)
  // bf16x6: every block reads its columns' weights for all of K, so the
  // weights cross L2 once per row block.  64-column blocks of two 16-row
  // tiles where 32-column ones would not all be resident at once (two 8-wave
  // blocks per CU); the second row tile halves the weight reads (C2 res512
  // k3 conv 19.8 -> 18.2 us, its 1x1 conv 9.6 -> 9.0 us against one tile).
  const bool wide = out_channels % 64 == 0 && (long)(out_channels / 32) * row_blocks > 512;
  const dim3 grid64(out_channels / 64, (unsigned)((rows + 31) / 32));
#define FM_ROWCONV64(KK) hipLaunchKernelGGL((row16_conv_kernel<KK, 64, true, 2>), grid64, dim3(512), 0, stream, p)
  const dim3 grid32r(out_channels / 32, (unsigned)((rows + 31) / 32));
#define FM_ROWCONV32R(KK) hipLaunchKernelGGL((row16_conv_kernel<KK, 32, true, 2>), grid32r, dim3(512), 0, stream, p)
  // Two 16-row tiles per block where the one-tile grid has two blocks per CU
  // and the 64-column form does not apply (the decoder's first conv: 25.2 ->
  // 21.1 us at C2; with fewer blocks the CUs left idle cost more than the
  // halved weight reads save).
  const bool two = !wide && (long)(out_channels / 32) * row_blocks >= 512;
  if ((flags & FM_WEIGHTS_X6) && two) {
    if (K == 256) FM_ROWCONV32R(256);
    else if (K == 1536) FM_ROWCONV32R(1536);
    else if (K == 2048) FM_ROWCONV32R(2048);
    else if (K == 3072) FM_ROWCONV32R(3072);
    else FM_ROWCONV32R(3584);
  } else if ((flags & FM_WEIGHTS_X6) && wide) {
    if (K == 256) FM_ROWCONV64(256);
    else if (K == 1536) FM_ROWCONV64(1536);
    else if (K == 2048) FM_ROWCONV64(2048);
    else if (K == 3072) FM_ROWCONV64(3072);
    else FM_ROWCONV64(3584);
  } else if (flags & FM_WEIGHTS_X6) {
    if (K == 256) FM_ROWCONV(256, true);
    else if (K == 1536) FM_ROWCONV(1536, true);
    else if (K == 2048) FM_ROWCONV(2048, true);
    else if (K == 3072) FM_ROWCONV(3072, true);
    else FM_ROWCONV(3584, true);
  } else {
    if (K == 1536) FM_ROWCONV(1536, false);
    else if (K == 2048) FM_ROWCONV(2048, false);
    else if (K == 3072) FM_ROWCONV(3072, false);
    else FM_ROWCONV(3584, false);
  }
#undef FM_ROWCONV
#undef FM_ROWCONV64
#undef FM_ROWCONV32R
  return (int)hipGetLastError();
}

}  // extern "C"
