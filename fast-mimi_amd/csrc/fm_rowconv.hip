// Few-row convolutions with long K: the 12.5 / 25 Hz end of the SEANet stacks
// at B x T <= 512 output rows (the encoder's last conv 1024 -> 512 k3, the
// bottleneck's replicate-padded downsample 512 -> 512 k4 s2, the decoder's
// first conv 512 -> 1024 k7).  The tiled GEMM engine has a few dozen tiles
// there and splits K across blocks with a second reduce launch; this kernel
// instead gives every 16 output rows x BN columns one block of 8 waves that
// split K, as the transformer's row-block projections do, and sums the 8
// partial tiles through LDS in wave order.
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
  const float* bias; // [N] or null
  float* y;          // [batch][rows_per_batch][N]
  int L, c_in, stride, pad_l, replicate, rows_per_batch, rows, N, flags;
};

template <int K, int BN>
__global__ __launch_bounds__(512) void row16_conv_kernel(RowConvArgs p) {
  constexpr int NWV = 8, BM = 16, KW = K / NWV, NP = KW / 64, NT = BN / 16;
  constexpr int PR = BN + 4, OPT = BM * BN / 512;
  static_assert(KW % 64 == 0 && OPT >= 1, "tile shape");
  __shared__ __attribute__((aligned(16))) float red[NWV * BM * PR];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const long m0 = (long)blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int kw0 = wave * KW;

  // This lane's output row (clamped: rows past the end load a valid row and
  // are not stored) and its window start.
  const long mr = min(m0 + li, (long)p.rows - 1);
  const int b = (int)(mr / p.rows_per_batch);
  const int t = (int)(mr - (long)b * p.rows_per_batch);
  const int p0 = t * p.stride - p.pad_l;
  const float* xb = p.x + (long)b * p.L * p.c_in + 16 * g;
  auto a_src = [&](int piece) -> const float* {
    const int k = kw0 + 64 * piece;  // wave-uniform
    const int tap = k / p.c_in;
    int pos = p0 + tap;
    if (p.replicate) pos = min(max(pos, 0), p.L - 1);
    else if ((unsigned)pos >= (unsigned)p.L) return g_zero_row;
    return xb + (long)pos * p.c_in + (k - tap * p.c_in);
  };
  const long tstride = (long)(K / 64) * 4 * 64 * 4;  // floats between 16-column tiles
  const float* wb = p.w + ((((long)(n0 / 16) * (K / 64) + kw0 / 64) * 4) * 64 + lane) * 4;
  const bool elu_in = p.flags & FM_ELU_IN;
  floatx4 a[2][4], bw[2][NT][4];
  auto load = [&](int buf, int piece) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int q = 0; q < 4; ++q)
        bw[buf][j][q] = *reinterpret_cast<const floatx4*>(wb + j * tstride + piece * 1024 + q * 256);
    const float* src = a_src(piece);
#pragma unroll
    for (int q = 0; q < 4; ++q) a[buf][q] = *reinterpret_cast<const floatx4*>(src + 4 * q);
  };

  floatx4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
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
          acc[j] = __builtin_amdgcn_mfma_f32_16x16x4f32(a[c][q][e], bw[c][j][q][e], acc[j], 0, 0, 0);
  }

  // The 8 partial tiles summed in wave order, then bias and the output ELU.
#pragma unroll
  for (int j = 0; j < NT; ++j)
#pragma unroll
    for (int r = 0; r < 4; ++r) red[(wave * BM + 4 * g + r) * PR + 16 * j + li] = acc[j][r];
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
    if (p.bias) v = __fadd_rn(v, p.bias[n0 + ec + c]);
    if (p.flags & FM_EPI_ELU) v = fm_elu(v);
    out[c] = v;
  }
  float* dst = p.y + m * p.N + n0 + ec;
#pragma unroll
  for (int c = 0; c < OPT; ++c) dst[c] = out[c];
}

}  // namespace

extern "C" {

int fm_conv1d_rows_supported(int in_channels, int out_channels, int kernel) {
  const int K = in_channels * kernel;
  return in_channels % 64 == 0 && out_channels % 32 == 0 && (K == 2048 || K == 3072 || K == 3584);
}

int fm_conv1d_rows(const float* x, int batch, int length, int in_channels,
                   const float* weight_rowpacked, const float* bias, int out_channels, int kernel,
                   int stride, int pad_mode, int flags, float* y, hipStream_t stream) {
  if (!x || !weight_rowpacked || !y || batch < 0 || length < 0 || kernel <= 0 || stride <= 0 ||
      kernel < stride || (pad_mode != 0 && pad_mode != 1))
    return FM_BAD_ARGUMENT;
  if (flags & ~(FM_ELU_IN | FM_EPI_ELU)) return FM_UNSUPPORTED;
  if (!fm_conv1d_rows_supported(in_channels, out_channels, kernel)) return FM_UNSUPPORTED;
  const int rows_per_batch = (length + stride - 1) / stride;
  const long rows = (long)batch * rows_per_batch;
  if (rows == 0) return FM_OK;
  if (length == 0) return FM_BAD_ARGUMENT;
  if ((rows + 15) / 16 > 65535) return FM_UNSUPPORTED;
  RowConvArgs p{x, weight_rowpacked, bias, y, length, in_channels, stride, kernel - stride, pad_mode,
                rows_per_batch, (int)rows, out_channels, flags};
  const dim3 grid(out_channels / 32, (unsigned)((rows + 15) / 16));
  const int K = in_channels * kernel;
  if (K == 2048) hipLaunchKernelGGL((row16_conv_kernel<2048, 32>), grid, dim3(512), 0, stream, p);
  else if (K == 3072) hipLaunchKernelGGL((row16_conv_kernel<3072, 32>), grid, dim3(512), 0, stream, p);
  else hipLaunchKernelGGL((row16_conv_kernel<3584, 32>), grid, dim3(512), 0, stream, p);
  return (int)hipGetLastError();
}

}  // extern "C"
