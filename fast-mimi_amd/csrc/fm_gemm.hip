// Implicit-GEMM engine for every dense contraction of the Mimi hot path:
// causal Conv1d (any kernel/stride, zero or replicate padding), causal
// ConvTranspose1d via stride-phase decomposition, and Linear layers, all on
// channels-last [batch, positions, channels] FP32 tensors with FP32 MFMA
// (v_mfma_f32_32x32x2f32) and fused epilogues (bias, ELU, GELU, residual add,
// LayerScale residual).
//
// The GEMM A operand is a *window view* of the input: output row m = (b, t)
// reads the contiguous run x[b, t*rs - padL : t*rs - padL + K/C_in, :], which
// in channels-last memory is K consecutive floats.  Positions outside [0, L)
// read zero (causal / stride-alignment padding) or clamp to the edge
// (replicate padding).  B is the packed weight [K, N] (row-major).

#include "fm_common.h"

namespace {

struct GemmArgs {
  const float* x;
  const float* w;
  const float* bias;
  const float* res;
  const float* scale;
  float* y;
  float* partial;
  int batch, L_in, C_in, rows, rs, padL, K, N, y_rows, bias_len, k_split, flags;
};

constexpr int BK = 32;

FM_DEVICE float epilogue(float v, long m, int n, const GemmArgs& p) {
  if (p.bias) v = __fadd_rn(v, p.bias[n % p.bias_len]);
  if (p.flags & FM_EPI_RES_ADD) v = __fadd_rn(p.res[m * p.N + n], v);
  if (p.flags & FM_EPI_RES_SCALE) v = __fadd_rn(p.res[m * p.N + n], __fmul_rn(p.scale[n], v));
  if (p.flags & FM_EPI_ELU) v = fm_elu(v);
  if (p.flags & FM_EPI_GELU) v = fm_gelu(v);
  return v;
}

FM_DEVICE void store_out(float acc, long m, int n, const GemmArgs& p) {
  const long b = m / p.rows;
  const long t = m - b * p.rows;
  if (t < p.y_rows) p.y[(b * p.y_rows + t) * p.N + n] = epilogue(acc, m, n, p);
}

template <int BM, int BN, int WM, int WN, int VA, int VB>
__global__ __launch_bounds__(64 * WM * WN) void gemm_kernel(GemmArgs p) {
  constexpr int NT = 64 * WM * WN;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int PA = BM + 1;  // As[k][m]: odd pitch keeps transposed writes conflict-light
  constexpr int PB = BN + 4;  // Bs[k][n]: 16-byte aligned rows
  constexpr int ACH = BM * BK / VA;  // A load chunks per tile
  constexpr int BCH = BK * BN / VB;
  constexpr int APT = (ACH + NT - 1) / NT;
  constexpr int BPT = (BCH + NT - 1) / NT;
  static_assert(FM >= 1 && FN >= 1, "wave tile must hold a 32x32 block");

  __shared__ float As[BK * PA];
  __shared__ float Bs[BK * PB];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int wm0 = (wave / WN) * WTM;
  const int wn0 = (wave % WN) * WTN;

  const long M = (long)p.batch * p.rows;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = blockIdx.x;
  const long m0 = (long)(tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;
  const int k_begin = blockIdx.y * p.k_split;
  const int k_end = min(p.K, k_begin + p.k_split);

  // Per-chunk row descriptors (fixed across the K loop).
  long a_off[APT];   // element offset of (b, p0) in x, p0 = first window position
  int a_p0[APT];     // first window position, -1e9 when the row is out of range
  int a_bL[APT];     // b * L_in
  int a_r[APT], a_k[APT];
#pragma unroll
  for (int i = 0; i < APT; ++i) {
    const int c = tid + i * NT;
    const int r = c / (BK / VA);
    const int kq = c % (BK / VA);
    a_r[i] = r;
    a_k[i] = kq * VA;
    const long m = m0 + r;
    if (c < ACH && m < M) {
      const long b = m / p.rows;
      const long t = m - b * p.rows;
      const int p0 = (int)(t * p.rs - p.padL);
      a_p0[i] = p0;
      a_bL[i] = (int)(b * p.L_in);
      a_off[i] = ((long)b * p.L_in + p0) * p.C_in;
    } else {
      a_p0[i] = -1000000000;
      a_bL[i] = 0;
      a_off[i] = 0;
    }
  }

  float ra[APT][VA];
  float rb[BPT][VB];

  auto load_a = [&](int k0) {
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int kg = k0 + a_k[i];
      bool ok = a_p0[i] > -1000000000 && kg < k_end;
      int pos = 0;
      if (ok) {
        pos = a_p0[i] + kg / p.C_in;
        if (p.flags & FM_REPLICATE) {
          pos = min(max(pos, 0), p.L_in - 1);
        } else {
          ok = pos >= 0 && pos < p.L_in;
        }
      }
      if (ok) {
        const float* src = (p.flags & FM_REPLICATE)
                               ? p.x + ((long)a_bL[i] + pos) * p.C_in + (kg % p.C_in)
                               : p.x + a_off[i] + kg;
        if constexpr (VA == 4) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(src);
          ra[i][0] = v.x; ra[i][1] = v.y; ra[i][2] = v.z; ra[i][3] = v.w;
        } else {
          ra[i][0] = *src;
        }
        if (p.flags & FM_ELU_IN) {
#pragma unroll
          for (int j = 0; j < VA; ++j) ra[i][j] = fm_elu(ra[i][j]);
        }
      } else {
#pragma unroll
        for (int j = 0; j < VA; ++j) ra[i][j] = 0.0f;
      }
    }
  };

  auto load_b = [&](int k0) {
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int c = tid + i * NT;
      const int kr = c / (BN / VB);
      const int nn = (c % (BN / VB)) * VB;
      const int kg = k0 + kr;
      const int n = n0 + nn;
      if (c < BCH && kg < k_end && n < p.N) {
        const float* src = p.w + (long)kg * p.N + n;
        if constexpr (VB == 4) {
          const floatx4 v = *reinterpret_cast<const floatx4*>(src);
          rb[i][0] = v.x; rb[i][1] = v.y; rb[i][2] = v.z; rb[i][3] = v.w;
        } else {
          rb[i][0] = *src;
        }
      } else {
#pragma unroll
        for (int j = 0; j < VB; ++j) rb[i][j] = 0.0f;
      }
    }
  };

  auto store_lds = [&]() {
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int c = tid + i * NT;
      if (c < ACH) {
#pragma unroll
        for (int j = 0; j < VA; ++j) As[(a_k[i] + j) * PA + a_r[i]] = ra[i][j];
      }
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int c = tid + i * NT;
      if (c < BCH) {
        const int kr = c / (BN / VB);
        const int nn = (c % (BN / VB)) * VB;
        if constexpr (VB == 4) {
          floatx4 v = {rb[i][0], rb[i][1], rb[i][2], rb[i][3]};
          *reinterpret_cast<floatx4*>(&Bs[kr * PB + nn]) = v;
        } else {
          Bs[kr * PB + nn] = rb[i][0];
        }
      }
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  if (k_begin < k_end) load_a(k_begin), load_b(k_begin);
  const int lrow = lane >> 5;
  const int lcol = lane & 31;
  for (int k0 = k_begin; k0 < k_end; k0 += BK) {
    __syncthreads();
    store_lds();
    __syncthreads();
    if (k0 + BK < k_end) {
      load_a(k0 + BK);
      load_b(k0 + BK);
    }
#pragma unroll
    for (int kk = 0; kk < BK; kk += 2) {
      float a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) a[i] = As[(kk + lrow) * PA + wm0 + i * 32 + lcol];
#pragma unroll
      for (int j = 0; j < FN; ++j) b[j] = Bs[(kk + lrow) * PB + wn0 + j * 32 + lcol];
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) acc[i][j] = fm_mfma32(a[i], b[j], acc[i][j]);
    }
  }

#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const long m = m0 + wm0 + i * 32 + fm_mfma32_row(r, lane);
        const int n = n0 + wn0 + j * 32 + lcol;
        if (m < M && n < p.N) {
          if (p.partial)
            p.partial[((long)blockIdx.y * M + m) * p.N + n] = acc[i][j][r];
          else
            store_out(acc[i][j][r], m, n, p);
        }
      }
}

// Sums split-K partials in split order and applies the epilogue.
__global__ __launch_bounds__(256) void splitk_reduce_kernel(GemmArgs p, int splits) {
  const long M = (long)p.batch * p.rows;
  const long total = M * p.N;
  for (long e = (long)blockIdx.x * blockDim.x + threadIdx.x; e < total;
       e += (long)gridDim.x * blockDim.x) {
    float s = p.partial[e];
    for (int k = 1; k < splits; ++k) s = __fadd_rn(s, p.partial[(long)k * total + e]);
    const long m = e / p.N;
    store_out(s, m, (int)(e - m * p.N), p);
  }
}

enum TileKind { TILE_N32, TILE_N64, TILE_BIG, TILE_SMALLM };

template <int BM, int BN, int WM, int WN>
hipError_t launch_cfg(GemmArgs p, int splits, hipStream_t s) {
  const long M = (long)p.batch * p.rows;
  const int tiles = (int)(((M + BM - 1) / BM) * ((p.N + BN - 1) / BN));
  dim3 grid(tiles, splits);
  dim3 block(64 * WM * WN);
  const bool va = (p.C_in % 4 == 0) && (p.K % 4 == 0) && !(p.flags & FM_REPLICATE && p.C_in % 4);
  const bool vb = (p.N % 4 == 0);
  if (va && vb) hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, 4, 4>), grid, block, 0, s, p);
  else if (va) hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, 4, 1>), grid, block, 0, s, p);
  else if (vb) hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, 1, 4>), grid, block, 0, s, p);
  else hipLaunchKernelGGL((gemm_kernel<BM, BN, WM, WN, 1, 1>), grid, block, 0, s, p);
  return hipGetLastError();
}

int run_gemm(GemmArgs p, float* workspace, size_t workspace_bytes, hipStream_t s) {
  if (!p.x || !p.w || !p.y || p.batch < 0 || p.rows < 0 || p.K <= 0 || p.N <= 0 ||
      p.C_in <= 0 || p.L_in < 0 || p.rs <= 0 || p.y_rows < 0 || p.y_rows > p.rows)
    return FM_BAD_ARGUMENT;
  if ((p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE)) && !p.res) return FM_BAD_ARGUMENT;
  if ((p.flags & FM_EPI_RES_SCALE) && !p.scale) return FM_BAD_ARGUMENT;
  if (p.bias && p.bias_len <= 0) return FM_BAD_ARGUMENT;
  const long M = (long)p.batch * p.rows;
  if (M == 0 || p.y_rows == 0) return FM_OK;
  if (p.L_in == 0) return FM_BAD_ARGUMENT;

  int BM, BN;
  TileKind kind;
  if (p.N <= 32) { kind = TILE_N32; BM = 128; BN = 32; }
  else if (p.N <= 64) { kind = TILE_N64; BM = 128; BN = 64; }
  else if (M <= 1024) { kind = TILE_SMALLM; BM = 32; BN = 128; }
  else { kind = TILE_BIG; BM = 128; BN = 128; }

  const long tiles = ((M + BM - 1) / BM) * ((p.N + BN - 1) / BN);
  const int ktiles = (p.K + BK - 1) / BK;
  int splits = 1;
  const long target = 1024;  // blocks to fill 256 CUs several times over
  if (tiles < target && ktiles >= 8 && workspace) {
    splits = (int)((target + tiles - 1) / tiles);
    splits = min(splits, ktiles / 4);
    splits = min(splits, 32);
    const size_t per = (size_t)M * p.N * sizeof(float);
    while (splits > 1 && per * splits > workspace_bytes) --splits;
    if (splits < 1) splits = 1;
  }
  p.k_split = ((ktiles + splits - 1) / splits) * BK;
  splits = (p.K + p.k_split - 1) / p.k_split;
  p.partial = splits > 1 ? workspace : nullptr;

  hipError_t e;
  switch (kind) {
    case TILE_N32: e = launch_cfg<128, 32, 4, 1>(p, splits, s); break;
    case TILE_N64: e = launch_cfg<128, 64, 4, 1>(p, splits, s); break;
    case TILE_SMALLM: e = launch_cfg<32, 128, 1, 4>(p, splits, s); break;
    default: e = launch_cfg<128, 128, 2, 2>(p, splits, s); break;
  }
  if (e != hipSuccess) return (int)e;
  if (splits > 1) {
    const long total = M * p.N;
    const int blocks = (int)min((total + 255) / 256, (long)4096);
    hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, p, splits);
    e = hipGetLastError();
  }
  return (int)e;
}

}  // namespace

extern "C" {

int fm_conv1d(const float* x, int batch, int length, int in_channels, const float* weight_packed,
              const float* bias, int out_channels, int kernel, int stride, int pad_mode, int flags,
              const float* residual, float* y, int y_length, float* workspace,
              size_t workspace_bytes, hipStream_t stream) {
  if (kernel <= 0 || stride <= 0 || kernel < stride || (pad_mode != 0 && pad_mode != 1))
    return FM_BAD_ARGUMENT;
  GemmArgs p{};
  p.x = x; p.w = weight_packed; p.bias = bias; p.res = residual; p.scale = nullptr; p.y = y;
  p.batch = batch; p.L_in = length; p.C_in = in_channels;
  p.rows = (length + stride - 1) / stride;  // ceil(L / stride): causal + stride-aligned
  p.rs = stride; p.padL = kernel - stride; p.K = kernel * in_channels; p.N = out_channels;
  p.y_rows = y_length; p.bias_len = out_channels;
  p.flags = (flags & ~FM_REPLICATE) | (pad_mode == 1 ? FM_REPLICATE : 0);
  if (p.flags & FM_EPI_RES_SCALE) return FM_BAD_ARGUMENT;
  return run_gemm(p, workspace, workspace_bytes, stream);
}

int fm_conv_transpose1d(const float* x, int batch, int length, int in_channels,
                        const float* weight_packed, const float* bias, int out_channels, int kernel,
                        int stride, int flags, const float* residual, float* y, float* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  if (kernel <= 0 || stride <= 0 || kernel % stride != 0) return FM_UNSUPPORTED;
  const int taps = kernel / stride;
  GemmArgs p{};
  p.x = x; p.w = weight_packed; p.bias = bias; p.res = residual; p.scale = nullptr; p.y = y;
  p.batch = batch; p.L_in = length; p.C_in = in_channels; p.rows = length; p.rs = 1;
  p.padL = taps - 1; p.K = taps * in_channels; p.N = stride * out_channels; p.y_rows = length;
  p.bias_len = out_channels; p.flags = flags & ~FM_REPLICATE;
  if (p.flags & FM_EPI_RES_SCALE) return FM_BAD_ARGUMENT;
  return run_gemm(p, workspace, workspace_bytes, stream);
}

int fm_linear(const float* x, int rows, int in_features, const float* weight_packed,
              int out_features, int flags, const float* residual, const float* scale, float* y,
              float* workspace, size_t workspace_bytes, hipStream_t stream) {
  GemmArgs p{};
  p.x = x; p.w = weight_packed; p.bias = nullptr; p.res = residual; p.scale = scale; p.y = y;
  p.batch = 1; p.L_in = rows; p.C_in = in_features; p.rows = rows; p.rs = 1; p.padL = 0;
  p.K = in_features; p.N = out_features; p.y_rows = rows; p.bias_len = 0;
  p.flags = flags & ~(FM_REPLICATE | FM_ELU_IN);
  return run_gemm(p, workspace, workspace_bytes, stream);
}

}  // extern "C"
