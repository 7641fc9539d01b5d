// Transformer pieces of the Mimi hot path that are not plain GEMMs:
//  * LayerNorm over the hidden dimension (one wave64 per row);
//  * causal sliding-window attention with RoPE applied as Q/K are staged,
//    reading Q, K, V straight out of the packed QKV projection and writing the
//    [rows, heads*head_dim] layout the output projection consumes.

#include "fm_common.h"

namespace {

FM_DEVICE float wave_sum(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  return v;
}

// y = (x - mean) * rstd * gamma + beta,  rstd = 1 / sqrt(var + eps) (biased var).
__global__ __launch_bounds__(256) void layer_norm_kernel(const float* __restrict__ x,
                                                         const float* __restrict__ gamma,
                                                         const float* __restrict__ beta, long rows,
                                                         int C, float eps, float* __restrict__ y) {
  const int lane = threadIdx.x & 63;
  const long row = (long)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (row >= rows) return;
  const float* xr = x + row * C;
  float s = 0.0f;
  for (int c = lane; c < C; c += 64) s += xr[c];
  const float mean = wave_sum(s) / (float)C;
  float v = 0.0f;
  for (int c = lane; c < C; c += 64) {
    const float d = xr[c] - mean;
    v = fmaf(d, d, v);
  }
  const float var = wave_sum(v) / (float)C;
  const float rstd = 1.0f / sqrtf(var + eps);
  float* yr = y + row * C;
  for (int c = lane; c < C; c += 64)
    yr[c] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(xr[c], mean), rstd), gamma[c]), beta[c]);
}

constexpr int QB = 32;  // queries per block (one MFMA column tile)
constexpr int KB = 32;  // keys per MFMA row tile
constexpr int NW = 4;   // waves per block; they split the key range

// RoPE as the reference writes it: x*cos + rotate_half(x)*sin, each product
// and the sum rounded separately.
FM_DEVICE float rope1(float x, float partner, int d, int half, float c, float s) {
  const float rot = d < half ? -partner : partner;
  return __fadd_rn(__fmul_rn(x, c), __fmul_rn(rot, s));
}

// Stages rows t0 .. t0+31 (rows past t_last read as zero) of one head of the
// packed projection into a transposed LDS tile dst[d * P + r], with RoPE
// applied unless cos_t is null (rows already rotated by their producer).  Each of the NTH cooperating threads owns N elements; all global
// loads are issued before any use so they overlap.
template <int N, int NTH, int D, int DP, int P>
FM_DEVICE void stage_rope_t(float* dst, int tid, const float* __restrict__ qkv, int ld, int col0,
                            const float* __restrict__ cos_t, const float* __restrict__ sin_t,
                            long base, int t0, int t_last) {
  constexpr int HALF = D / 2;
  float x[N], xp[N], c[N], sn[N];
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int e = tid + u * NTH;
    const int r = e / DP, d = e % DP;
    const int t = t0 + r;
    x[u] = xp[u] = c[u] = sn[u] = 0.0f;
    if (t <= t_last && d < D) {
      const float* row = qkv + (base + t) * ld + col0;
      x[u] = row[d];
      if (cos_t) {
        xp[u] = row[d < HALF ? d + HALF : d - HALF];
        c[u] = cos_t[(long)t * D + d];
        sn[u] = sin_t[(long)t * D + d];
      }
    }
  }
#pragma unroll
  for (int u = 0; u < N; ++u) {
    const int e = tid + u * NTH;
    const int r = e / DP, d = e % DP;
    dst[d * P + r] = cos_t ? rope1(x[u], xp[u], d, HALF, c[u], sn[u]) : x[u];
  }
}

// Sliding-window causal attention on FP32 MFMA.
// Grid: (ceil(T / QB), heads, batch), 256 threads.  Block = 32 queries of one
// head; its key range [q0 - window + 1, q0 + 31] is cut into 32-key tiles that
// the 4 waves take round-robin, one tile per wave per round.  Q (once) and
// each wave's K tile are staged through LDS with row-contiguous loads and RoPE
// applied on the way in, stored transposed ([dim][32], odd pitch).  Per tile a
// wave computes S^T = K Q^T (keys on MFMA rows, queries on columns, lane l
// owns query q0 + l % 32), applies the window mask and an online softmax per
// column, then accumulates O^T += V^T P^T with P^T fed straight from the S^T
// registers: MFMA step s takes keys 8*(s/4) + 4*h + s%4 (h = lane / 32),
// exactly the rows that lane holds in accumulator slot s.  V is read straight
// from global memory (lanes read consecutive dims).  The waves' (max, sum, O)
// are merged through LDS.
template <int D>
__global__ __launch_bounds__(256) void window_attention_kernel(
    const float* __restrict__ qkv, int ld, int q_off, int k_off, int v_off,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int T, int heads,
    int kv_heads, int window, float scale, float* __restrict__ out, int ld_out) {
  constexpr int DT = (D + 31) / 32;  // 32-row tiles of O^T
  constexpr int DP = DT * 32;        // padded head dim
  constexpr int KS = DP / 2;         // MFMA k-steps of the QK^T product
  constexpr int HALF = D / 2;
  constexpr int P = QB + 1;          // pitch of the transposed [dim][32] tiles
  // Region 0: per-wave K tiles during the loop, per-wave O^T at the merge.
  __shared__ float stage[NW][DP * P];
  __shared__ float Qt[DP * P];
  __shared__ float Mm[NW][QB];
  __shared__ float Lm[NW][QB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int head = blockIdx.y;
  const int hk = head / (heads / kv_heads);
  const long b = blockIdx.z;
  const int q0 = blockIdx.x * QB;
  const int q = q0 + col;
  const int k_lo = max(0, q0 - window + 1);
  const int k_hi = min(T, q0 + QB) - 1;
  const long base = b * (long)T;

  // Stage Q^T with RoPE (zero for padded dims / rows past T).
  stage_rope_t<QB * DP / 256, 256, D, DP, P>(Qt, tid, qkv, ld, q_off + head * D, cos_t, sin_t,
                                            base, q0, T - 1);
  __syncthreads();
  float qv[KS];
#pragma unroll
  for (int i = 0; i < KS; ++i) qv[i] = Qt[(2 * i + h) * P + col];

  float m_run = -INFINITY, l_run = 0.0f;
  floatx16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;

  float* Kt = stage[wave];
  const int ntiles = (k_hi - k_lo + KB) / KB;
  const int rounds = (ntiles + NW - 1) / NW;
  for (int round = 0; round < rounds; ++round) {
    const int tile = round * NW + wave;
    const int k0 = k_lo + tile * KB;
    const bool active = tile < ntiles;
    __syncthreads();  // previous round's reads of Kt are done
    if (active)
      stage_rope_t<KB * DP / 64, 64, D, DP, P>(Kt, lane, qkv, ld, k_off + hk * D, cos_t, sin_t,
                                              base, k0, k_hi);
    __syncthreads();
    if (!active) continue;

    floatx16 s;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < KS; ++i) s = fm_mfma32(Kt[(2 * i + h) * P + col], qv[i], s);

    float cmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = k0 + fm_mfma32_row(r, lane);
      const bool ok = q < T && key <= k_hi && key <= q && key > q - window;
      s[r] = ok ? s[r] * scale : -INFINITY;
      cmax = fmaxf(cmax, s[r]);
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float m_new = fmaxf(m_run, cmax);
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const float pv = (s[r] == -INFINITY) ? 0.0f : expf(s[r] - m_new);
      s[r] = pv;
      psum += pv;
    }
    psum += __shfl_xor(psum, 32, 64);
    const float corr = (m_run == -INFINITY) ? 0.0f : expf(m_run - m_new);
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int t = 0; t < DT; ++t)
#pragma unroll
      for (int r = 0; r < 16; ++r) o[t][r] *= corr;
#pragma unroll
    for (int st = 0; st < 16; ++st) {
      const int key = k0 + 8 * (st >> 2) + 4 * h + (st & 3);
      const bool vok = key <= k_hi;
      const float* vrow = qkv + (base + (vok ? key : k_lo)) * ld + v_off + hk * D;
#pragma unroll
      for (int t = 0; t < DT; ++t) {
        const int d = t * 32 + col;
        const float vv = (vok && d < D) ? vrow[d] : 0.0f;
        o[t] = fm_mfma32(vv, s[st], o[t]);
      }
    }
  }

  // Merge the waves: O = sum_w O_w exp(m_w - M), L = sum_w l_w exp(m_w - M).
  __syncthreads();
  float* Om = stage[wave];
  if (h == 0) Mm[wave][col] = m_run, Lm[wave][col] = l_run;
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) Om[(t * 32 + fm_mfma32_row(r, lane)) * P + col] = o[t][r];
  __syncthreads();
  for (int e = tid; e < QB * D; e += 256) {
    const int qi = e / D, d = e % D;
    const int qg = q0 + qi;
    if (qg >= T) continue;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, Mm[w][qi]);
    float num = 0.0f, den = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      if (Mm[w][qi] == -INFINITY) continue;
      const float f = expf(Mm[w][qi] - M);
      num += stage[w][d * P + qi] * f;
      den += Lm[w][qi] * f;
    }
    out[(base + qg) * ld_out + head * D + d] = num / den;
  }
}


// Row-block linear layer for the transformer projections (K = hidden = 512):
//   y = epilogue( LN?(x) . W^T )
// A block of NWV waves owns 32 rows x BN output columns.  Its 32 input rows
// are loaded once, TPR = 2*NWV consecutive lanes per row; when gamma is given
// the LayerNorm statistics are reduced from those registers with lane
// shuffles and the rows are normalised before they are written to LDS, so the
// LayerNorm costs no launch or LDS pass of its own.  The waves split K; each
// wave fetches its weight fragments straight from global memory into
// registers (all issued before any use), so no staging or barrier sits in the
// MFMA loop.  The k-slot of lane half h at step 4q+e carries k = 16h + 4q + e,
// matching 16-byte LDS reads of A.  Partial tiles are summed through LDS in
// wave order, then the epilogue applies, per flag: RoPE (x*cos +
// rotate_half(x)*sin within each 64-wide head, for columns < rope_cols; needs
// BN == 64), exact GELU, or y = res + scale * acc.
template <int K, int BN, int NWV>
__global__ __launch_bounds__(64 * NWV) void row_linear_kernel(
    const float* __restrict__ x, int rows, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, const float* __restrict__ w, int N, int flags,
    const float* res, const float* __restrict__ scale, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int rope_cols, int rows_per_seq, float* y) {
  constexpr int BM = 32, NTH = 64 * NWV, PA = K + 4, KW = K / NWV, KT = KW / 32, NJ = BN / 32;
  constexpr int PR = BN + 4, TPR = NTH / BM, CH = K / 4 / TPR, OPT = BM * BN / NTH;
  static_assert(KW % 32 == 0 && CH >= 1 && OPT % 2 == 0, "tile shape");
  extern __shared__ __attribute__((aligned(16))) float sm[];
  float* As = sm;   // [BM][PA]
  float* red = sm;  // after the MFMAs: [NWV][BM][PR]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  const long m0 = (long)blockIdx.x * BM;
  const int n0 = blockIdx.y * BN;
  const int kw0 = wave * KW;

  // Weight fragments for this wave's k-slice.
  floatx4 bw[NJ][KT][4];
#pragma unroll
  for (int j = 0; j < NJ; ++j) {
    const float* wr = w + (long)(n0 + j * 32 + lcol) * K + kw0 + 16 * h;
#pragma unroll
    for (int kt = 0; kt < KT; ++kt)
#pragma unroll
      for (int q = 0; q < 4; ++q) bw[j][kt][q] = *reinterpret_cast<const floatx4*>(wr + kt * 32 + 4 * q);
  }
  // Row r = tid / TPR; lane part p holds float4 chunks p, p + TPR, ...
  {
    const int r = tid / TPR, p = tid % TPR;
    const bool valid = m0 + r < rows;
    const float* xr = x + min(m0 + r, (long)rows - 1) * K;
    floatx4 v[CH];
#pragma unroll
    for (int u = 0; u < CH; ++u) v[u] = *reinterpret_cast<const floatx4*>(xr + 4 * (p + TPR * u));
    if (gamma) {
      floatx4 gv[CH], bv[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        gv[u] = *reinterpret_cast<const floatx4*>(gamma + 4 * (p + TPR * u));
        bv[u] = *reinterpret_cast<const floatx4*>(beta + 4 * (p + TPR * u));
      }
      float s = 0.0f;
#pragma unroll
      for (int u = 0; u < CH; ++u) s += (v[u][0] + v[u][1]) + (v[u][2] + v[u][3]);
#pragma unroll
      for (int o = 1; o < TPR; o <<= 1) s += __shfl_xor(s, o, 64);
      const float mean = s / (float)K;
      float var = 0.0f;
#pragma unroll
      for (int u = 0; u < CH; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float d = v[u][e] - mean;
          var = fmaf(d, d, var);
        }
#pragma unroll
      for (int o = 1; o < TPR; o <<= 1) var += __shfl_xor(var, o, 64);
      const float rstd = 1.0f / sqrtf(var / (float)K + eps);
#pragma unroll
      for (int u = 0; u < CH; ++u)
#pragma unroll
        for (int e = 0; e < 4; ++e)
          v[u][e] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[u][e], mean), rstd), gv[u][e]), bv[u][e]);
    }
#pragma unroll
    for (int u = 0; u < CH; ++u)
      *reinterpret_cast<floatx4*>(As + r * PA + 4 * (p + TPR * u)) =
          valid ? v[u] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
  __syncthreads();

  floatx16 acc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
#pragma unroll
  for (int kt = 0; kt < KT; ++kt)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const floatx4 a = *reinterpret_cast<const floatx4*>(As + lcol * PA + kw0 + kt * 32 + 16 * h + 4 * q);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < NJ; ++j) acc[j] = fm_mfma32(a[e], bw[j][kt][q][e], acc[j]);
    }
  __syncthreads();  // all waves are done with As; reuse it for the partial tiles
#pragma unroll
  for (int j = 0; j < NJ; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) red[(wave * BM + fm_mfma32_row(r, lane)) * PR + j * 32 + lcol] = acc[j][r];
  __syncthreads();
  // Sum the partial tiles in wave order (OPT consecutive outputs per thread).
  const int er = tid / TPR, ec = (tid % TPR) * OPT;
  float out[OPT];
#pragma unroll
  for (int c = 0; c < OPT; ++c) {
    float v = red[er * PR + ec + c];
#pragma unroll
    for (int g = 1; g < NWV; ++g) v = __fadd_rn(v, red[(g * BM + er) * PR + ec + c]);
    out[c] = v;
  }
  const long m = m0 + er;
  const bool rope = BN == 64 && cos_t && n0 < rope_cols;
  if (rope) {
    __syncthreads();
#pragma unroll
    for (int c = 0; c < OPT; ++c) red[er * PR + ec + c] = out[c];
    __syncthreads();
  }
  if (m >= rows) return;
  const int t = (int)(m % rows_per_seq);
#pragma unroll
  for (int c = 0; c < OPT; ++c) {
    const int n = n0 + ec + c;
    float v = out[c];
    if (rope) {
      const int d = ec + c;  // dim within the 64-wide head
      const float partner = red[er * PR + (d < 32 ? d + 32 : d - 32)];
      const float rot = d < 32 ? -partner : partner;
      v = __fadd_rn(__fmul_rn(v, cos_t[(long)t * 64 + d]), __fmul_rn(rot, sin_t[(long)t * 64 + d]));
    }
    if (flags & FM_EPI_GELU) v = fm_gelu(v);
    if (flags & FM_EPI_RES_SCALE) v = __fadd_rn(res[m * N + n], __fmul_rn(scale[n], v));
    out[c] = v;
  }
  float* dst = y + m * N + n0 + ec;
#pragma unroll
  for (int c = 0; c < OPT; c += 2) *reinterpret_cast<float2*>(dst + c) = float2{out[c], out[c + 1]};
}

}  // namespace

extern "C" {

// Transformer projection with optional fused LayerNorm prologue (gamma/beta
// non-null), RoPE epilogue on columns < rope_cols (cos/sin non-null; head_dim
// 64, tables [rows_per_seq][64]), GELU or LayerScale-residual epilogue.
// in_features must be 512 (Mimi's hidden width); out_features a multiple of 64.
int fm_row_linear_supported(int in_features, int out_features) {
  return in_features == 512 && out_features % 64 == 0;
}

int fm_row_linear(const float* x, int rows, int in_features, const float* ln_gamma,
                  const float* ln_beta, float ln_eps, const float* weight, int out_features,
                  int flags, const float* residual, const float* scale, const float* rope_cos,
                  const float* rope_sin, int rope_cols, int rows_per_seq, float* y,
                  hipStream_t stream) {
  if (!x || !weight || !y || rows < 0 || rows_per_seq <= 0 || (ln_gamma && !ln_beta))
    return FM_BAD_ARGUMENT;
  if (!fm_row_linear_supported(in_features, out_features)) return FM_UNSUPPORTED;
  if ((flags & FM_EPI_RES_SCALE) && (!residual || !scale)) return FM_BAD_ARGUMENT;
  if (rope_cos && (!rope_sin || rope_cols % 64)) return FM_BAD_ARGUMENT;
  if (rows == 0) return FM_OK;
  constexpr int K = 512;
  // 64-wide column tiles where RoPE needs whole heads, else 32-wide tiles (twice the blocks,
  // half the MFMA chain per wave); 8 waves split K.
  const bool wide = rope_cos != nullptr;
#define FM_ROWLIN(BN, NWV)                                                                       \
  {                                                                                              \
    const size_t lds = std::max<size_t>((size_t)32 * (K + 4), (size_t)NWV * 32 * (BN + 4)) * 4;  \
    hipLaunchKernelGGL((row_linear_kernel<K, BN, NWV>), dim3((rows + 31) / 32, out_features / BN), \
                       dim3(64 * NWV), lds, stream, x, rows, ln_gamma, ln_beta, ln_eps, weight,   \
                       out_features, flags, residual, scale, rope_cos, rope_sin, rope_cols,      \
                       rows_per_seq, y);                                                         \
  }
  if (wide)
    FM_ROWLIN(64, 8)
  else
    FM_ROWLIN(32, 8)
#undef FM_ROWLIN
  return (int)hipGetLastError();
}

int fm_layer_norm(const float* x, const float* gamma, const float* beta, long rows, int channels,
                  float eps, float* y, hipStream_t stream) {
  if (!x || !gamma || !beta || !y || rows < 0 || channels <= 0) return FM_BAD_ARGUMENT;
  if (rows == 0) return FM_OK;
  const long blocks = (rows + 3) / 4;
  hipLaunchKernelGGL(layer_norm_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, gamma,
                     beta, rows, channels, eps, y);
  return (int)hipGetLastError();
}

int fm_window_attention(const float* qkv, int ld_qkv, int q_offset, int k_offset, int v_offset,
                        const float* cos_table, const float* sin_table, int batch, int length,
                        int heads, int kv_heads, int head_dim, int window, float scale, float* out,
                        int ld_out, hipStream_t stream) {
  if (!qkv || !cos_table != !sin_table || !out || batch < 0 || length < 0 || heads <= 0 ||
      kv_heads <= 0 || heads % kv_heads || window <= 0)
    return FM_BAD_ARGUMENT;
  if (batch == 0 || length == 0) return FM_OK;
  dim3 grid((length + QB - 1) / QB, heads, batch);
#define FM_ATT(DV)                                                                          \
  hipLaunchKernelGGL(window_attention_kernel<DV>, grid, dim3(256), 0, stream, qkv, ld_qkv,  \
                     q_offset, k_offset, v_offset, cos_table, sin_table, length, heads,     \
                     kv_heads, window, scale, out, ld_out)
  switch (head_dim) {
    case 8: FM_ATT(8); break;
    case 16: FM_ATT(16); break;
    case 32: FM_ATT(32); break;
    case 64: FM_ATT(64); break;
    default: return FM_UNSUPPORTED;
  }
#undef FM_ATT
  return (int)hipGetLastError();
}

}  // extern "C"
