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

// LayerNorm for C = 512: 32 lanes per row, each holding float4 chunks
// p, p + 32, p + 64, p + 96 of it, so the row is read once and the
// statistics come from registers.  The arithmetic (per-lane partial sums,
// shuffle order, two-pass variance) is the one of the LayerNorm prologue of
// row16_linear_kernel, so both paths round identically.
__global__ __launch_bounds__(256) void layer_norm512_kernel(const float* __restrict__ x,
                                                            const float* __restrict__ gamma,
                                                            const float* __restrict__ beta,
                                                            long rows, float eps,
                                                            float* __restrict__ y) {
  constexpr int K = 512, TPR = 32, CH = K / 4 / TPR;
  const long row = (long)blockIdx.x * 8 + (threadIdx.x >> 5);
  const int p = threadIdx.x & 31;
  const float* xr = x + min(row, rows - 1) * K;
  floatx4 v[CH], gv[CH], bv[CH];
#pragma unroll
  for (int u = 0; u < CH; ++u) v[u] = *reinterpret_cast<const floatx4*>(xr + 4 * (p + TPR * u));
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
  if (row >= rows) return;
  float* yr = y + row * K;
#pragma unroll
  for (int u = 0; u < CH; ++u) {
    floatx4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e)
      o[e] = __fadd_rn(__fmul_rn(__fmul_rn(__fsub_rn(v[u][e], mean), rstd), gv[u][e]), bv[u][e]);
    *reinterpret_cast<floatx4*>(yr + 4 * (p + TPR * u)) = o;
  }
}

FM_DEVICE floatx4 fm_mfma16(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// One v_mfma_f32_16x16x32_bf16: lane l supplies row / column l % 16 at
// k = 8 (l / 16) .. +7; results as fm_mfma16.
FM_DEVICE floatx4 fm_mfma16_bf16(bf16x8 a, bf16x8 b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

constexpr int QB = 32;  // queries per block (one MFMA column tile)
constexpr int KB = 32;  // keys per MFMA row tile

// RoPE as the reference writes it: x*cos + rotate_half(x)*sin, each product
// and the sum rounded separately.  For the pair (x_d, x_{d+half}) with the
// shared angle (cos, sin): lo' = lo*c - hi*s, hi' = hi*c + lo*s.
FM_DEVICE void rope_pair(floatx4& lo, floatx4& hi, const floatx4& c, const floatx4& s) {
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const float l = lo[e], u = hi[e];
    lo[e] = __fadd_rn(__fmul_rn(l, c[e]), __fmul_rn(-u, s[e]));
    hi[e] = __fadd_rn(__fmul_rn(u, c[e]), __fmul_rn(l, s[e]));
  }
}

// Rows t0 .. t0+31 of one head of Q or K (D dims, row pitch ld), held as
// float4 pairs (dims 4c.. and 4c + D/2..) so that RoPE's partners sit in the
// same lane; rows past t_last read as zero.  NTH threads share the tile.
template <int D, int NTH, bool ROPE, int ROWS = QB>
struct RowTile {
  static constexpr int HALF = D / 2, PAIRS = ROWS * D / 8;
  static constexpr int N = (PAIRS + NTH - 1) / NTH;
  floatx4 lo[N], hi[N], c[N], s[N];
  unsigned okm;  // rows inside the sequence; zeroing waits for the store (see VTile)

  FM_DEVICE void load(int tid, const float* __restrict__ src, long ld, int t0, int t_last,
                      const float* __restrict__ cos_t, const float* __restrict__ sin_t) {
    okm = 0;
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int e = tid + u * NTH;
      const int r = e / (D / 8), d = (e % (D / 8)) * 4;
      const int t = min(t0 + r, t_last);
      okm |= (unsigned)(e < PAIRS && t0 + r <= t_last) << u;
      const float* row = src + (long)t * ld;
      lo[u] = *reinterpret_cast<const floatx4*>(row + d);
      hi[u] = *reinterpret_cast<const floatx4*>(row + d + HALF);
      if (ROPE) {
        c[u] = *reinterpret_cast<const floatx4*>(cos_t + (long)t * D + d);
        s[u] = *reinterpret_cast<const floatx4*>(sin_t + (long)t * D + d);
      }
    }
  }
  // Writes the tile to dst[row * pitch + dim], rotated when ROPE.
  FM_DEVICE void store(int tid, float* dst, int pitch) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int e = tid + u * NTH;
      if (PAIRS % NTH && e >= PAIRS) continue;
      const int r = e / (D / 8), d = (e % (D / 8)) * 4;
      const bool ok = (okm >> u) & 1;
      floatx4 l = ok ? lo[u] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      floatx4 h = ok ? hi[u] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (ROPE) rope_pair(l, h, c[u], s[u]);
      *reinterpret_cast<floatx4*>(dst + r * pitch + d) = l;
      *reinterpret_cast<floatx4*>(dst + r * pitch + d + HALF) = h;
    }
  }
};

// V rows t0 .. t0+31 (zero past t_last and in the padded dims D..DP).
template <int D, int DP>
struct VTile {
  static constexpr int CHUNKS = QB * DP / 4, N = (CHUNKS + 63) / 64;
  floatx4 v[N];
  // Validity bits; the zeroing select is applied at the store, so a prefetch
  // does not wait for its loads where it is issued.
  unsigned okm;
  FM_DEVICE void load(int lane, const float* __restrict__ src, long ld, int t0, int t_last) {
    okm = 0;
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int e = lane + u * 64;
      const int r = e / (DP / 4), d = (e % (DP / 4)) * 4;
      const int t = min(t0 + r, t_last);
      v[u] = *reinterpret_cast<const floatx4*>(src + (long)t * ld + min(d, D - 4));
      okm |= (unsigned)(e < CHUNKS && t0 + r <= t_last && d < D) << u;
    }
  }
  FM_DEVICE void store(int lane, float* dst, int pitch) {
#pragma unroll
    for (int u = 0; u < N; ++u) {
      const int e = lane + u * 64;
      if (CHUNKS % 64 && e >= CHUNKS) continue;
      const int r = e / (DP / 4), d = (e % (DP / 4)) * 4;
      *reinterpret_cast<floatx4*>(dst + r * pitch + d) =
          ((okm >> u) & 1) ? v[u] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    }
  }
};

// Sliding-window causal attention on FP32 MFMA.
// Grid: (ceil((T - q_start) / QB), heads, batch), 64 * NW threads.  Queries are
// rows q_start .. T-1 (earlier rows are cached keys/values only); query q
// writes output row q - q_start.  Block = 32 queries of one
// head; its key range [q0 - window + 1, q0 + 31] is cut into 32-key tiles that
// the NW waves take round-robin.  Waves run independently after the shared Q
// stage: each keeps its next K/V tile in flight in registers while it
// computes on the current one from its own LDS slot (rows contiguous, K pitch
// D+4, V pitch DP+8).  Per tile a wave computes S^T = K Q^T (keys on MFMA
// rows, queries on columns, lane l owns query q0 + l % 32; the k-slot of lane
// half h at step 4j+e carries dim D/2*h + 4j + e so both operands come from
// 16-byte LDS reads), applies the window mask and an online softmax per
// column, then accumulates O^T += V^T P^T with P^T fed straight from the S^T
// registers: MFMA step s takes keys 8*(s/4) + 4*h + s%4, exactly the rows
// that lane holds in accumulator slot s.  The waves' (max, sum, O) are merged
// through LDS.  ROPE: rotate Q and K while staging (else they arrive rotated).
template <int D, bool ROPE, int NW>
__global__ __launch_bounds__(64 * NW) void window_attention_kernel(
    const float* __restrict__ qkv, int ld, int q_off, int k_off, int v_off,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int T, int q_start,
    int heads, int kv_heads, int window, float scale, float* __restrict__ out, int ld_out) {
  constexpr int NTH = 64 * NW;
  constexpr int DT = (D + 31) / 32;  // 32-row tiles of O^T
  constexpr int DP = DT * 32;        // padded head dim of V / O
  constexpr int PK = D + 4, PV = DP + 8, P = QB + 1;
  constexpr int SLOT = QB * PK + KB * PV;  // per-wave K + V tile
  static_assert(DP * P <= SLOT, "merge tile fits the slot");
  __shared__ __attribute__((aligned(16))) float stage[NW][SLOT];
  __shared__ __attribute__((aligned(16))) float Qs[QB * PK];
  __shared__ float Mm[NW][QB];
  __shared__ float Lm[NW][QB];
  __shared__ float Fm[NW][QB];
  __shared__ float Dm[QB];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, col = lane & 31;
  const int head = blockIdx.y;
  const int hk = head / (heads / kv_heads);
  const long b = blockIdx.z;
  const int q0 = q_start + blockIdx.x * QB;
  const int q = q0 + col;
  const int k_lo = max(0, q0 - window + 1);
  const int k_hi = min(T, q0 + QB) - 1;
  const float* seq = qkv + b * (long)T * ld;
  const float* kcol = seq + k_off + hk * D;
  const float* vcol = seq + v_off + hk * D;

  const int ntiles = (k_hi - k_lo + KB) / KB;
  RowTile<D, 64, ROPE> kr;
  VTile<D, DP> vr;
  if (wave < ntiles) {
    kr.load(lane, kcol, ld, k_lo + wave * KB, k_hi, cos_t, sin_t);
    vr.load(lane, vcol, ld, k_lo + wave * KB, k_hi);
  }
  {
    RowTile<D, NTH, ROPE> qr;
    qr.load(tid, seq + q_off + head * D, ld, q0, T - 1, cos_t, sin_t);
    qr.store(tid, Qs, PK);
  }
  __syncthreads();
  float qv[D / 2];
#pragma unroll
  for (int j = 0; j < D / 8; ++j) {
    const floatx4 t4 = *reinterpret_cast<const floatx4*>(Qs + col * PK + (D / 2) * h + 4 * j);
#pragma unroll
    for (int e = 0; e < 4; ++e) qv[4 * j + e] = t4[e];
  }

  float m_run = -INFINITY, l_run = 0.0f;
  floatx16 o[DT];
#pragma unroll
  for (int t = 0; t < DT; ++t)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[t][r] = 0.0f;

  float* Ks = stage[wave];
  float* Vs = Ks + QB * PK;
  for (int tile = wave; tile < ntiles; tile += NW) {
    const int k0 = k_lo + tile * KB;
    kr.store(lane, Ks, PK);
    vr.store(lane, Vs, PV);
    wave_lds_fence();
    if (tile + NW < ntiles) {  // next tile's loads overlap this tile's math
      kr.load(lane, kcol, ld, k0 + NW * KB, k_hi, cos_t, sin_t);
      vr.load(lane, vcol, ld, k0 + NW * KB, k_hi);
    }

    // Two interleaved MFMA chains (even / odd 4-dim groups), summed after.
    floatx16 s, s2;
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] = 0.0f, s2[r] = 0.0f;
#pragma unroll
    for (int j = 0; j < D / 8; ++j) {
      const floatx4 a4 = *reinterpret_cast<const floatx4*>(Ks + col * PK + (D / 2) * h + 4 * j);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        if (j & 1) s2 = fm_mfma32(a4[e], qv[4 * j + e], s2);
        else s = fm_mfma32(a4[e], qv[4 * j + e], s);
      }
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) s[r] += s2[r];

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
      const float* vrow = Vs + (8 * (st >> 2) + 4 * h + (st & 3)) * PV + col;
#pragma unroll
      for (int t = 0; t < DT; ++t) o[t] = fm_mfma32(vrow[t * 32], s[st], o[t]);
    }
    wave_lds_fence();  // this tile's LDS reads are done before the slot is rewritten
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
  // Per query: M = max_w m_w, the factors f_w = exp(m_w - M) (0 for a wave
  // that saw no key) and den = sum_w l_w f_w, once; then each output element
  // is sum_w O_w f_w / den.
  if (tid < QB) {
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, Mm[w][tid]);
    float den = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = (Mm[w][tid] == -INFINITY) ? 0.0f : expf(Mm[w][tid] - M);
      Fm[w][tid] = f;
      if (Mm[w][tid] != -INFINITY) den += Lm[w][tid] * f;
    }
    Dm[tid] = den;
  }
  __syncthreads();
  for (int e = tid; e < QB * D; e += NTH) {
    const int qi = e / D, d = e % D;
    const int qg = q0 + qi;
    if (qg >= T) continue;
    float num = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w)
      if (Mm[w][qi] != -INFINITY) num += stage[w][d * P + qi] * Fm[w][qi];
    out[(b * (long)(T - q_start) + qg - q_start) * ld_out + head * D + d] = num / Dm[qi];
  }
}


// Sliding-window causal attention for head_dim 64 on 16x16x4 FP32 MFMA.
// Block = 16 queries of one head (twice the blocks of the 32-query kernel, so
// short sequences spread over more CUs; the per-block MFMA work is what bounds
// this kernel at a few hundred frames).  The key range is cut into 32-key
// tiles taken round-robin by the NW waves, each with its own LDS slot and the
// next tile's K/V prefetched in registers.  Per tile a wave forms S^T = K Q^T
// as two 16-key row tiles (lane (g, i) = (l / 16, l % 16) owns query i and
// keys 4g..4g+3 of each; k-slot g at step 4t+e carries dim 16g + 4t + e, so K
// comes from 16-byte LDS reads and Q^T from registers), four MFMA chains
// (row tile x even/odd t).  After the window mask and an online softmax per
// query, O^T += V^T P^T runs with P^T straight from the S^T registers: step r
// of row tile kt uses key 16kt + 4g + r in k-slot g, exactly the key that
// lane holds in accumulator slot r.  O^T is four 16-dim row tiles (four
// chains).  The waves' (max, sum, O) are merged through LDS with the factors
// exp(m_w - M) computed once per query.  ROPE: Q and K rotate while staging.
template <bool ROPE, int NW>
__global__ __launch_bounds__(64 * NW) void window_attention16_kernel(
    const float* __restrict__ qkv, int ld, int q_off, int k_off, int v_off,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int T, int q_start,
    int heads, int kv_heads, int window, float scale, float* __restrict__ out, int ld_out) {
  constexpr int D = 64, QT = 16, NTH = 64 * NW;
  constexpr int PK = D + 4, PVV = D + 4, P = QT + 1;
  constexpr int SLOT = KB * PK + KB * PVV;
  static_assert(D * P <= SLOT, "merge tile fits the slot");
  __shared__ __attribute__((aligned(16))) float stage[NW][SLOT];
  __shared__ __attribute__((aligned(16))) float Qs[ROPE ? QT * PK : 4];
  __shared__ float Mm[NW][QT];
  __shared__ float Lm[NW][QT];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int head = blockIdx.y;
  const int hk = head / (heads / kv_heads);
  const long b = blockIdx.z;
  const int q0 = q_start + blockIdx.x * QT;
  const int q = q0 + i;
  const int k_lo = max(0, q0 - window + 1);
  const int k_hi = min(T, q0 + QT) - 1;
  const float* seq = qkv + b * (long)T * ld;
  const float* kcol = seq + k_off + hk * D;
  const float* vcol = seq + v_off + hk * D;

  const int ntiles = (k_hi - k_lo + KB) / KB;
  RowTile<D, 64, ROPE> kr;
  VTile<D, D> vr;
  if (wave < ntiles) {
    kr.load(lane, kcol, ld, k_lo + wave * KB, k_hi, cos_t, sin_t);
    vr.load(lane, vcol, ld, k_lo + wave * KB, k_hi);
  }
  float qv[16];  // query i, dims 16g .. 16g+15
  if constexpr (ROPE) {
    // RoPE pairs dims d and d +- 32: the tile is rotated while staged in LDS.
    RowTile<D, NTH, ROPE, QT> qr;
    qr.load(tid, seq + q_off + head * D, ld, q0, T - 1, cos_t, sin_t);
    qr.store(tid, Qs, PK);
    __syncthreads();
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const floatx4 t4 = *reinterpret_cast<const floatx4*>(Qs + i * PK + 16 * g + 4 * t);
#pragma unroll
      for (int e = 0; e < 4; ++e) qv[4 * t + e] = t4[e];
    }
  } else {
    // Each wave reads its query fragments straight from memory: no LDS pass
    // and no block barrier before the key loop.
    const float* qrow = seq + (long)min(q, T - 1) * ld + q_off + head * D + 16 * g;
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const floatx4 t4 = *reinterpret_cast<const floatx4*>(qrow + 4 * t);
#pragma unroll
      for (int e = 0; e < 4; ++e) qv[4 * t + e] = t4[e];
    }
  }

  // Scores are kept in base-2 units (scale * log2 e folded in) so every
  // exponential is one hardware exp2.
  const float scale2 = scale * 1.44269504088896341f;
  float m_run = -INFINITY, l_run = 0.0f;
  floatx4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  float* Ks = stage[wave];
  float* Vs = Ks + KB * PK;
  for (int tile = wave; tile < ntiles; tile += NW) {
    const int k0 = k_lo + tile * KB;
    kr.store(lane, Ks, PK);
    vr.store(lane, Vs, PVV);
    wave_lds_fence();
    if (tile + NW < ntiles) {  // next tile's loads overlap this tile's math
      kr.load(lane, kcol, ld, k0 + NW * KB, k_hi, cos_t, sin_t);
      vr.load(lane, vcol, ld, k0 + NW * KB, k_hi);
    }

    floatx4 sc[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int par = 0; par < 2; ++par) sc[kt][par] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const floatx4 a4 = *reinterpret_cast<const floatx4*>(Ks + (16 * kt + i) * PK + 16 * g + 4 * t);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[kt][t & 1] = fm_mfma16(a4[e], qv[4 * t + e], sc[kt][t & 1]);
      }
    float sv[2][4];
    float cmax = -INFINITY;
    // A tile whose keys lie inside every query's window (and the sequence)
    // needs no per-score mask: only the diagonal and window-edge tiles do.
    const bool full = q0 + QT <= T && k0 + KB - 1 <= k_hi && k0 + KB - 1 <= q0 &&
                      k0 > q0 + QT - 1 - window;
    if (full) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sv[kt][r] = (sc[kt][0][r] + sc[kt][1][r]) * scale2;
          cmax = fmaxf(cmax, sv[kt][r]);
        }
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 16 * kt + 4 * g + r;
          const bool ok = q < T && key <= k_hi && key <= q && key > q - window;
          const float v = sc[kt][0][r] + sc[kt][1][r];
          sv[kt][r] = ok ? v * scale2 : -INFINITY;
          cmax = fmaxf(cmax, sv[kt][r]);
        }
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float m_new = fmaxf(m_run, cmax);
    // exp2(-inf) = 0 covers masked scores; a query with nothing unmasked yet
    // subtracts 0 instead of -inf so no -inf - -inf NaN forms.
    const float m_sub = m_new == -INFINITY ? 0.0f : m_new;
    float psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(sv[kt][r] - m_sub);
        sv[kt][r] = pv;
        psum += pv;
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(m_run - m_sub);
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[dt][r] *= corr;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vrow = Vs + (16 * kt + 4 * g + r) * PVV + i;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = fm_mfma16(vrow[16 * dt], sv[kt][r], o[dt]);
      }
    wave_lds_fence();  // this tile's LDS reads are done before the slot is rewritten
  }

  // Merge the waves: O = sum_w O_w f_w / sum_w l_w f_w, f_w = 2^(m_w - M), m in base-2 units.
  // Each wave parks its running state in its own slot (its key-loop reads of
  // that slot are fenced above), so one barrier suffices; every output
  // element then forms the factors of its query in wave order.
  float* Om = stage[wave];
  if (g == 0) Mm[wave][i] = m_run, Lm[wave][i] = l_run;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) Om[(16 * dt + 4 * g + r) * P + i] = o[dt][r];
  __syncthreads();
  for (int e = tid; e < QT * D; e += NTH) {
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
      const float f = __builtin_amdgcn_exp2f(Mm[w][qi] - M);
      num += stage[w][d * P + qi] * f;
      den += Lm[w][qi] * f;
    }
    out[(b * (long)(T - q_start) + qg - q_start) * ld_out + head * D + d] = num / den;
  }
}


// Long-sequence attention for head_dim 64 (hundreds to thousands of frames,
// few sequence-heads): block = 16 * NWQ consecutive queries of one head, NWQ
// waves, wave w owning queries q0 + 16w .. +15.  The block's key range
// [q0 - window + 1, q0 + 16 NWQ - 1] streams through LDS in 32-key chunks (K
// rotated while staged when ROPE), double-buffered from a one-chunk register
// prefetch, one barrier per chunk, so each key row is fetched once per block
// instead of once per 16 queries.  Each wave runs the online softmax of
// window_attention16_kernel over the chunks that meet its own window and
// writes its rows; no cross-wave merge.  Several blocks share a CU (35 KB of
// LDS each).  Measured at 2500 frames: two waves per block (32 queries) 35 us
// per layer, four 36 us, one 50 us (the 16-query kernel: 47.5 us); 64- or
// 128-key chunks are slower (their register prefetch spills).
template <bool ROPE, int NWQ>
__global__ __launch_bounds__(64 * NWQ) void window_attention_flash_kernel(
    const float* __restrict__ qkv, int ld, int q_off, int k_off, int v_off,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int T, int q_start,
    int heads, int kv_heads, int window, float scale, float* __restrict__ out, int ld_out) {
  constexpr int D = 64, QT = 16, QBLK = QT * NWQ, NTH = 64 * NWQ, PK = D + 4, PV = D + 4;
  constexpr int CK = KB;  // keys per chunk
  constexpr int STAGE = CK * (PK + PV);
  constexpr int KPT = CK * (D / 8) / NTH, VPT = CK * (D / 4) / NTH;  // K pairs / V chunks per thread
  static_assert(KPT >= 1 && VPT >= 1, "chunk loader");
  __shared__ __attribute__((aligned(16))) float lds[2 * STAGE];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int head = blockIdx.y;
  const int hk = head / (heads / kv_heads);
  const long b = blockIdx.z;
  const int q0 = q_start + blockIdx.x * QBLK;
  const int q0w = q0 + QT * wave;
  const int q = q0w + i;
  const float* seq = qkv + b * (long)T * ld;
  const float* kcol = seq + k_off + hk * D;
  const float* vcol = seq + v_off + hk * D;
  const int kb_lo = max(0, q0 - window + 1);
  const int kb_hi = min(T, q0 + QBLK) - 1;
  const int nch = (kb_hi - kb_lo + CK) / CK;
  const bool live = q0w < T;
  const int wk_lo = max(0, q0w - window + 1);
  const int wk_hi = min(T, q0w + QT) - 1;

  // Chunk loader: K pair e = tid + u * NTH is row e / 8, dims 4(e % 8) and
  // +32; V chunk e = tid + u * NTH is row e / 16, dims 4(e % 16).
  floatx4 klo[KPT], khi[KPT], kc[KPT], ks[KPT], vv[VPT];
  auto load = [&](int k0) {
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int e = tid + u * NTH, kr = e >> 3, kd = (e & 7) * 4;
      const int t = min(k0 + kr, kb_hi);
      klo[u] = *reinterpret_cast<const floatx4*>(kcol + (long)t * ld + kd);
      khi[u] = *reinterpret_cast<const floatx4*>(kcol + (long)t * ld + kd + D / 2);
      if (ROPE) {
        kc[u] = *reinterpret_cast<const floatx4*>(cos_t + (long)t * D + kd);
        ks[u] = *reinterpret_cast<const floatx4*>(sin_t + (long)t * D + kd);
      }
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int e = tid + u * NTH;
      vv[u] = *reinterpret_cast<const floatx4*>(vcol + (long)min(k0 + e / 16, kb_hi) * ld + (e % 16) * 4);
    }
  };
  auto store = [&](int stage) {
    float* Ks = lds + stage * STAGE;
    float* Vs = Ks + CK * PK;
#pragma unroll
    for (int u = 0; u < KPT; ++u) {
      const int e = tid + u * NTH, kr = e >> 3, kd = (e & 7) * 4;
      floatx4 l = klo[u], hh = khi[u];
      if (ROPE) rope_pair(l, hh, kc[u], ks[u]);
      *reinterpret_cast<floatx4*>(Ks + kr * PK + kd) = l;
      *reinterpret_cast<floatx4*>(Ks + kr * PK + kd + D / 2) = hh;
    }
#pragma unroll
    for (int u = 0; u < VPT; ++u) {
      const int e = tid + u * NTH;
      *reinterpret_cast<floatx4*>(Vs + (e / 16) * PV + (e % 16) * 4) = vv[u];
    }
  };

  load(kb_lo);
  // Query i of this wave, dims 16g .. 16g+15, rotated in registers.
  float qv[16];
  {
    const int qc = min(q, T - 1);
    const float* qrow = seq + (long)qc * ld + q_off + head * D;
#pragma unroll
    for (int t4 = 0; t4 < 4; ++t4) {
      const int d = 16 * g + 4 * t4;
      floatx4 x = *reinterpret_cast<const floatx4*>(qrow + d);
      if (ROPE) {
        const int dl = d & (D / 2 - 1);
        const floatx4 y = *reinterpret_cast<const floatx4*>(qrow + (d ^ (D / 2)));
        const floatx4 c = *reinterpret_cast<const floatx4*>(cos_t + (long)qc * D + dl);
        const floatx4 sn = *reinterpret_cast<const floatx4*>(sin_t + (long)qc * D + dl);
        floatx4 lo = d < D / 2 ? x : y, hi = d < D / 2 ? y : x;
        rope_pair(lo, hi, c, sn);
        x = d < D / 2 ? lo : hi;
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) qv[4 * t4 + e] = x[e];
    }
  }

  const float scale2 = scale * 1.44269504088896341f;
  float m_run = -INFINITY, l_run = 0.0f;
  floatx4 o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) o[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  for (int c = 0; c < nch; ++c) {
    const int kc0 = kb_lo + c * CK;
    store(c & 1);
    __syncthreads();  // chunk c staged; every wave is past its reads of chunk c - 2
    if (c + 1 < nch) load(kc0 + CK);
    const int k0 = kc0;
    if (!live || k0 > wk_hi || k0 + KB - 1 < wk_lo) continue;
    const float* Kt = lds + (c & 1) * STAGE;
    const float* Vt = Kt + CK * PK;
    floatx4 sc[2][2];
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int par = 0; par < 2; ++par) sc[kt][par] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int kt = 0; kt < 2; ++kt) {
        const floatx4 a4 = *reinterpret_cast<const floatx4*>(Kt + (16 * kt + i) * PK + 16 * g + 4 * t);
#pragma unroll
        for (int e = 0; e < 4; ++e) sc[kt][t & 1] = fm_mfma16(a4[e], qv[4 * t + e], sc[kt][t & 1]);
      }
    float sv[2][4];
    float cmax = -INFINITY;
    const bool full = q0w + QT <= T && k0 + KB - 1 <= wk_hi && k0 + KB - 1 <= q0w &&
                      k0 > q0w + QT - 1 - window;
    if (full) {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sv[kt][r] = (sc[kt][0][r] + sc[kt][1][r]) * scale2;
          cmax = fmaxf(cmax, sv[kt][r]);
        }
    } else {
#pragma unroll
      for (int kt = 0; kt < 2; ++kt)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int key = k0 + 16 * kt + 4 * g + r;
          const bool ok = q < T && key <= kb_hi && key <= q && key > q - window;
          const float v = sc[kt][0][r] + sc[kt][1][r];
          sv[kt][r] = ok ? v * scale2 : -INFINITY;
          cmax = fmaxf(cmax, sv[kt][r]);
        }
    }
    cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
    cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
    const float m_new = fmaxf(m_run, cmax);
    const float m_sub = m_new == -INFINITY ? 0.0f : m_new;
    float psum = 0.0f;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float pv = __builtin_amdgcn_exp2f(sv[kt][r] - m_sub);
        sv[kt][r] = pv;
        psum += pv;
      }
    psum += __shfl_xor(psum, 16, 64);
    psum += __shfl_xor(psum, 32, 64);
    const float corr = __builtin_amdgcn_exp2f(m_run - m_sub);
    l_run = l_run * corr + psum;
    m_run = m_new;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) o[dt][r] *= corr;
#pragma unroll
    for (int kt = 0; kt < 2; ++kt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const float* vrow = Vt + (16 * kt + 4 * g + r) * PV + i;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt) o[dt] = fm_mfma16(vrow[16 * dt], sv[kt][r], o[dt]);
      }
  }
  if (!live || q >= T) return;
  float* orow = out + (b * (long)(T - q_start) + q - q_start) * ld_out + head * D;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int r = 0; r < 4; ++r) orow[16 * dt + 4 * g + r] = o[dt][r] / l_run;
}

constexpr int SEQ_MAX = 256;
// Whole-sequence attention for head_dim 64 and sequences of at most 256
// frames (the batched 12.5-25 Hz transformers): one block per (half, head,
// sequence) stages the head's K (rotated when ROPE) and V for every frame in
// LDS once, so no key row is fetched twice by a block.  The 16 query tiles of
// 16 frames are paired (j, 15 - j) so that every pair costs the same number
// of key tiles under the causal mask; block half s owns pairs 4s .. 4s+3.
// NKS waves share a pair and take its key tiles round-robin; each keeps both
// of its query tiles' (max, sum, O) in registers and the pair merges once at
// the end, parking the states over the staged K/V.  The inner step is the one
// of window_attention16_kernel: S^T = K Q^T on 16x16x4 MFMA with K from
// 16-byte LDS reads and Q^T from registers, an online softmax in base-2
// units, and O^T += V^T P^T with P^T from the S^T registers.  A key tile may
// run up to 31 rows past the staged frames; those rows are masked.
// Measured at C3 (B 16, 250 frames): 25.8 us per layer with NKS = 2; 27.2 us
// with NKS = 3; 28.6 us when the pair merged after each query tile.
template <bool ROPE, int NKS>
__global__ __launch_bounds__(256 * NKS) void window_attention_seq_kernel(
    const float* __restrict__ qkv, int ld, int q_off, int k_off, int v_off,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int T, int heads,
    int kv_heads, int window, float scale, float* __restrict__ out, int ld_out) {
  constexpr int D = 64, QT = 16, PK = D + 4, PV = D + 4, P = QT + 1, NTH = 256 * NKS;
  constexpr int PARK = D * P + 2 * QT;  // one parked (O^T, max, sum)
  static_assert(4 * (NKS - 1) * 2 * PARK <= SEQ_MAX * (PV + PK), "states park over K/V");
  // V, then K, then 32 rows that absorb the masked reads of a key tile that
  // runs past the staged frames (V overruns read K rows).
  __shared__ __attribute__((aligned(16))) float lds[SEQ_MAX * (PV + PK) + KB * PK];
  float* Vs = lds;                 // [SEQ_MAX][PV]
  float* Ks = Vs + SEQ_MAX * PV;    // [SEQ_MAX][PK]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, i = lane & 15;
  const int pair = wave & 3, kh = wave >> 2;
  const int head = blockIdx.y;
  const int hk = head / (heads / kv_heads);
  const long b = blockIdx.z;
  const float* seq = qkv + b * (long)T * ld;

  {
    constexpr int PAIRS = SEQ_MAX * D / 8, KN = (PAIRS + NTH - 1) / NTH;
    const float* kcol = seq + k_off + hk * D;
#pragma unroll
    for (int u = 0; u < KN; ++u) {
      const int e = tid + u * NTH;
      if (PAIRS % NTH && e >= PAIRS) break;
      const int r = e / (D / 8), d = (e % (D / 8)) * 4;
      const int t = min(r, T - 1);
      floatx4 lo = *reinterpret_cast<const floatx4*>(kcol + (long)t * ld + d);
      floatx4 hi = *reinterpret_cast<const floatx4*>(kcol + (long)t * ld + d + D / 2);
      if (r >= T) lo = hi = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (ROPE) {
        const floatx4 c = *reinterpret_cast<const floatx4*>(cos_t + (long)t * D + d);
        const floatx4 sn = *reinterpret_cast<const floatx4*>(sin_t + (long)t * D + d);
        rope_pair(lo, hi, c, sn);
      }
      *reinterpret_cast<floatx4*>(Ks + r * PK + d) = lo;
      *reinterpret_cast<floatx4*>(Ks + r * PK + d + D / 2) = hi;
    }
    constexpr int CH = SEQ_MAX * D / 4, VN = (CH + NTH - 1) / NTH;
    const float* vcol = seq + v_off + hk * D;
#pragma unroll
    for (int u = 0; u < VN; ++u) {
      const int e = tid + u * NTH;
      if (CH % NTH && e >= CH) break;
      const int r = e / (D / 4), d = (e % (D / 4)) * 4;
      floatx4 v = *reinterpret_cast<const floatx4*>(vcol + (long)min(r, T - 1) * ld + d);
      if (r >= T) v = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      *reinterpret_cast<floatx4*>(Vs + r * PV + d) = v;
    }
  }
  __syncthreads();

  const float scale2 = scale * 1.44269504088896341f;
  const int jp = blockIdx.x * 4 + pair;
  float m_st[2], l_st[2];
  floatx4 o_st[2][4];
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int qt = half == 0 ? jp : 15 - jp;
    const int q0 = qt * QT;
    const bool live = q0 < T;
    const int q = q0 + i;
    float m_run = -INFINITY, l_run = 0.0f;
    floatx4 o[4];
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o[dt] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    if (live) {
      float qv[16];
      const float* qrow = seq + (long)min(q, T - 1) * ld + q_off + head * D;
#pragma unroll
      for (int t4 = 0; t4 < 4; ++t4) {
        const int d = 16 * g + 4 * t4;
        floatx4 x = *reinterpret_cast<const floatx4*>(qrow + d);
        if (ROPE) {
          const int dl = d & (D / 2 - 1);
          const floatx4 y = *reinterpret_cast<const floatx4*>(qrow + (d ^ (D / 2)));
          const floatx4 c = *reinterpret_cast<const floatx4*>(cos_t + (long)min(q, T - 1) * D + dl);
          const floatx4 sn = *reinterpret_cast<const floatx4*>(sin_t + (long)min(q, T - 1) * D + dl);
          floatx4 lo = d < D / 2 ? x : y, hi = d < D / 2 ? y : x;
          rope_pair(lo, hi, c, sn);
          x = d < D / 2 ? lo : hi;
        }
#pragma unroll
        for (int e = 0; e < 4; ++e) qv[4 * t4 + e] = x[e];
      }
      const int k_lo = max(0, q0 - window + 1);
      const int k_hi = min(T, q0 + QT) - 1;
      const int ntiles = (k_hi - k_lo + KB) / KB;
      for (int tile = kh; tile < ntiles; tile += NKS) {
        const int k0 = k_lo + tile * KB;
        const float* Kt = Ks + k0 * PK;
        const float* Vt = Vs + k0 * PV;
        floatx4 sc[2][2];
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int par = 0; par < 2; ++par) sc[kt][par] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int t = 0; t < 4; ++t)
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            const floatx4 a4 = *reinterpret_cast<const floatx4*>(Kt + (16 * kt + i) * PK + 16 * g + 4 * t);
#pragma unroll
            for (int e = 0; e < 4; ++e) sc[kt][t & 1] = fm_mfma16(a4[e], qv[4 * t + e], sc[kt][t & 1]);
          }
        float sv[2][4];
        float cmax = -INFINITY;
        const bool full = q0 + QT <= T && k0 + KB - 1 <= k_hi && k0 + KB - 1 <= q0 &&
                          k0 > q0 + QT - 1 - window;
        if (full) {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              sv[kt][r] = (sc[kt][0][r] + sc[kt][1][r]) * scale2;
              cmax = fmaxf(cmax, sv[kt][r]);
            }
        } else {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int key = k0 + 16 * kt + 4 * g + r;
              const bool ok = q < T && key <= k_hi && key <= q && key > q - window;
              const float v = sc[kt][0][r] + sc[kt][1][r];
              sv[kt][r] = ok ? v * scale2 : -INFINITY;
              cmax = fmaxf(cmax, sv[kt][r]);
            }
        }
        cmax = fmaxf(cmax, __shfl_xor(cmax, 16, 64));
        cmax = fmaxf(cmax, __shfl_xor(cmax, 32, 64));
        const float m_new = fmaxf(m_run, cmax);
        const float m_sub = m_new == -INFINITY ? 0.0f : m_new;
        float psum = 0.0f;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float pv = __builtin_amdgcn_exp2f(sv[kt][r] - m_sub);
            sv[kt][r] = pv;
            psum += pv;
          }
        psum += __shfl_xor(psum, 16, 64);
        psum += __shfl_xor(psum, 32, 64);
        const float corr = __builtin_amdgcn_exp2f(m_run - m_sub);
        l_run = l_run * corr + psum;
        m_run = m_new;
#pragma unroll
        for (int dt = 0; dt < 4; ++dt)
#pragma unroll
          for (int r = 0; r < 4; ++r) o[dt][r] *= corr;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt)
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float* vrow = Vt + (16 * kt + 4 * g + r) * PV + i;
#pragma unroll
            for (int dt = 0; dt < 4; ++dt) o[dt] = fm_mfma16(vrow[16 * dt], sv[kt][r], o[dt]);
          }
      }
    }
    m_st[half] = m_run;
    l_st[half] = l_run;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt) o_st[half][dt] = o[dt];
  }
  // Merge: waves kh > 0 park their two states over the K/V (every wave is
  // done reading them after this barrier); wave kh = 0 of each pair combines
  // O = sum_w O_w f_w / sum_w l_w f_w, f_w = 2^(m_w - M), in key-split order.
  __syncthreads();
  if (kh > 0) {
#pragma unroll
    for (int half = 0; half < 2; ++half) {
      float* pk = lds + ((pair * (NKS - 1) + kh - 1) * 2 + half) * PARK;
      if (g == 0) pk[D * P + i] = m_st[half], pk[D * P + QT + i] = l_st[half];
#pragma unroll
      for (int dt = 0; dt < 4; ++dt)
#pragma unroll
        for (int r = 0; r < 4; ++r) pk[(16 * dt + 4 * g + r) * P + i] = o_st[half][dt][r];
    }
  }
  __syncthreads();
  if (kh > 0) return;
#pragma unroll
  for (int half = 0; half < 2; ++half) {
    const int qt = half == 0 ? jp : 15 - jp;
    const int q = qt * QT + i;
    if (qt * QT >= T || q >= T) continue;
    float M = m_st[half];
#pragma unroll
    for (int w = 1; w < NKS; ++w) M = fmaxf(M, lds[((pair * (NKS - 1) + w - 1) * 2 + half) * PARK + D * P + i]);
    const float f0 = m_st[half] == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(m_st[half] - M);
    float den = l_st[half] * f0;
    float fw[NKS];
#pragma unroll
    for (int w = 1; w < NKS; ++w) {
      const float* pk = lds + ((pair * (NKS - 1) + w - 1) * 2 + half) * PARK;
      const float mw = pk[D * P + i];
      fw[w] = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f(mw - M);
      den += pk[D * P + QT + i] * fw[w];
    }
    float* orow = out + (b * (long)T + q) * ld_out + head * D;
#pragma unroll
    for (int dt = 0; dt < 4; ++dt)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int d = 16 * dt + 4 * g + r;
        float num = o_st[half][dt][r] * f0;
#pragma unroll
        for (int w = 1; w < NKS; ++w) num += lds[((pair * (NKS - 1) + w - 1) * 2 + half) * PARK + d * P + i] * fw[w];
        orow[d] = num / den;
      }
  }
}

// Grids of the row-block kernels put the column block in blockIdx.x: blocks
// are dealt round-robin to the 8 XCDs, so each XCD's L2 holds a slice of the
// weights (read once) plus the small activation block, instead of every XCD
// streaming all of the weights.
//
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
  // PR = 8 mod 16: the two lane halves (4 rows apart) store 32 banks apart.
  constexpr int PR = BN + 8, TPR = NTH / BM, CH = K / 4 / TPR, OPT = BM * BN / NTH;
  static_assert(KW % 32 == 0 && CH >= 1 && OPT % 2 == 0, "tile shape");
  extern __shared__ __attribute__((aligned(16))) float sm[];
  float* As = sm;   // [BM][PA]
  float* red = sm;  // after the MFMAs: [NWV][BM][PR]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  const long m0 = (long)blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
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


// Row-block linear layer for long K (K a multiple of 8 * 64, no LayerNorm):
// y = epilogue(x . W^T).  A block of 8 waves owns 32 rows x 32 columns; wave w
// takes k-range [w*K/8, (w+1)*K/8) in 64-dim pieces whose A and B fragments
// are loaded straight from global memory into registers one piece ahead of
// their use (lane half h at step 4j+e carries dim 32h + 4j + e of the piece,
// so every load is 16 bytes).  The 8 partial tiles are summed through LDS in
// wave order; epilogue GELU or y = res + scale * acc.
template <int K>
__global__ __launch_bounds__(512) void row_stream_linear_kernel(
    const float* __restrict__ x, int rows, const float* __restrict__ w, int N, int flags,
    const float* res, const float* __restrict__ scale, float* y) {
  // PR = 8 mod 16: the two lane halves (4 rows apart) store 32 banks apart.
  constexpr int NWV = 8, KW = K / NWV, NP = KW / 64, PR = 40;
  static_assert(KW % 64 == 0, "whole 64-dim pieces per wave");
  __shared__ float red[NWV * 32 * PR];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int h = lane >> 5, lcol = lane & 31;
  const long m0 = (long)blockIdx.y * 32;
  const int n0 = blockIdx.x * 32;
  const float* xr = x + min(m0 + lcol, (long)rows - 1) * K + wave * KW + 32 * h;
  const float* wr = w + (long)(n0 + lcol) * K + wave * KW + 32 * h;
  floatx4 a[2][8], b[2][8];
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    a[0][j] = *reinterpret_cast<const floatx4*>(xr + 4 * j);
    b[0][j] = *reinterpret_cast<const floatx4*>(wr + 4 * j);
  }
  __builtin_amdgcn_sched_barrier(0);
  floatx16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
  for (int p = 0; p < NP; ++p) {
    const int c = p & 1;
    if (p + 1 < NP) {
#pragma unroll
      for (int j = 0; j < 8; ++j) {
        a[c ^ 1][j] = *reinterpret_cast<const floatx4*>(xr + 64 * (p + 1) + 4 * j);
        b[c ^ 1][j] = *reinterpret_cast<const floatx4*>(wr + 64 * (p + 1) + 4 * j);
      }
    }
    __builtin_amdgcn_sched_barrier(0);  // keep the next piece's loads ahead of these MFMAs
#pragma unroll
    for (int j = 0; j < 8; ++j)
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fm_mfma32(a[c][j][e], b[c][j][e], acc);
  }
#pragma unroll
  for (int r = 0; r < 16; ++r) red[(wave * 32 + fm_mfma32_row(r, lane)) * PR + lcol] = acc[r];
  __syncthreads();
  // 1024 outputs, 2 per thread (adjacent columns).
  const int er = tid >> 4, ec = (tid & 15) * 2;
  const long m = m0 + er;
  if (m >= rows) return;
  float out[2];
#pragma unroll
  for (int c = 0; c < 2; ++c) {
    float v = red[er * PR + ec + c];
#pragma unroll
    for (int g = 1; g < NWV; ++g) v = __fadd_rn(v, red[(g * 32 + er) * PR + ec + c]);
    const int n = n0 + ec + c;
    if (flags & FM_EPI_GELU) v = fm_gelu(v);
    if (flags & FM_EPI_RES_SCALE) v = __fadd_rn(res[m * N + n], __fmul_rn(scale[n], v));
    out[c] = v;
  }
  *reinterpret_cast<float2*>(y + m * N + n0 + ec) = float2{out[0], out[1]};
}


// ---------------------------------------------------------------------------
// Packed row-block projections for few rows (the B x T <= ~512 transformer
// and RVQ projections): 16 rows x BN columns per block on the 16x16x4 FP32
// MFMA, 8 waves splitting K, so even 250 rows give hundreds of blocks.
// Weights are pre-packed (fm_pack_row_weights) in fragment order: the float4
// at index ((nt * (K/64) + kp) * 4 + t) * 64 + lane holds
// W[16 nt + lane % 16][64 kp + 16 (lane / 16) + 4 t .. + 3], so each wave
// load is 1 KB contiguous.  In a 64-dim piece the k-slot of lane group
// g = lane / 16 at MFMA step 4t+e carries dim 16 g + 4 t + e, for A as for B.
// K == 512: the 16 input rows are staged in LDS (and layer-normalised from
// registers when gamma is given: 32 lanes per row, shuffle-reduced).
// K == 2048: A fragments are streamed from global memory (no LayerNorm).
// Both double-buffer the next 64-dim piece in registers.  The 8 partial tiles
// are summed through LDS in wave order; epilogue as in row_linear_kernel.


// X6: the weight is W^T's bf16x6 planes ([3][K/16][N][16], fm_split_weights)
// and the contraction runs on v_mfma_f32_16x16x32_bf16 as the six cross
// terms of three-piece splits (FP32-accurate, see fm_gemm.hip): in a 32-deep
// k step, lane group g covers k = 8g .. 8g + 7 of A and B, the A fragment is
// split as it is read, and each B fragment of a plane is a 512-byte run.
// 1.85x the FP32 16x16x4 MFMA rate per contraction (measured 13.4 vs 18.5 ns
// per instruction, six against eight per 16 x 16 x 32).
//
// UPS: the projection feeds the depthwise ConvTranspose1d (kernel 4, stride
// 2, trim 2) of the decoder's upsample, y[2t + p] = h[t-1] w[p+2] + h[t] w[p]
// per channel (h[t-1] = 0 at a sequence start), computed in the epilogue: a
// block's 16 rows are t0 - 1 .. t0 + 14 (the first one only feeds row t0's
// taps), and y is the upsampled [rows * 2][N]; up_w is [N][4].
template <int K, int BN, bool X6 = false, bool UPS = false>
__global__ __launch_bounds__(512) void row16_linear_kernel(
    const float* __restrict__ x, int rows, const float* __restrict__ gamma,
    const float* __restrict__ beta, float eps, const float* __restrict__ wp, int N, int flags,
    const float* res, const float* __restrict__ scale, const float* __restrict__ cos_t,
    const float* __restrict__ sin_t, int rope_cols, int rows_per_seq, float* y,
    const float* __restrict__ up_w = nullptr) {
  constexpr int NWV = 8, BM = 16, KW = K / NWV, NP = KW / 64, NT = BN / 16;
  static_assert(!UPS || (!X6 && K == 512), "upsample epilogue on the staged FP32 path");
  constexpr bool STAGE = (K == 512);
  // PR = 4 mod 16: the four 16-lane groups of a partial-tile store hit disjoint banks.
  constexpr int PA = K + 4, PR = BN + 4, OPT = BM * BN / 512;
  static_assert(KW % 64 == 0 && OPT >= 1, "tile shape");
  constexpr int A_FLOATS = STAGE ? BM * PA : 0, R_FLOATS = NWV * BM * PR;
  __shared__ __attribute__((aligned(16))) float sm[A_FLOATS > R_FLOATS ? A_FLOATS : R_FLOATS];
  float* As = sm;
  float* red = sm;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = lane >> 4, li = lane & 15;
  const long m0 = UPS ? (long)blockIdx.y * (BM - 1) - 1 : (long)blockIdx.y * BM;
  const int n0 = blockIdx.x * BN;
  const int kw0 = wave * KW;

  // The 16 input rows into LDS, layer-normalised when gamma is given (32
  // lanes per row, float4 chunks p, p + 32, ..., shuffle-reduced).
  auto stage_rows = [&]() {
    constexpr int TPR = 32, CH = K / 4 / TPR;
    const int r = tid / TPR, p = tid % TPR;
    const bool valid = m0 + r < rows && m0 + r >= 0;
    const float* xr = x + max(min(m0 + r, (long)rows - 1), 0L) * K;
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
  };

  // Epilogue operands (residual, LayerScale, RoPE tables), fetched before
  // the MFMAs so their latency hides under them instead of trailing the
  // reduction.
  const int er = tid / (BN / OPT), ec = (tid % (BN / OPT)) * OPT;
  const long m = m0 + er;
  const long mc = max(min(m, (long)rows - 1), 0L);
  const int tpos = (int)(mc % rows_per_seq);
  const bool rope = BN == 64 && cos_t && n0 < rope_cols;
  const bool res_scale = flags & FM_EPI_RES_SCALE;
  float e_res[OPT], e_scale[OPT], e_cos[OPT], e_sin[OPT];
  auto fetch_epilogue = [&]() {
#pragma unroll
    for (int c = 0; c < OPT; ++c) {
      const int n = n0 + ec + c;
      e_res[c] = res_scale ? res[mc * N + n] : 0.0f;
      e_scale[c] = res_scale ? scale[n] : 0.0f;
      e_cos[c] = rope ? cos_t[(long)tpos * 64 + ec + c] : 0.0f;
      e_sin[c] = rope ? sin_t[(long)tpos * 64 + ec + c] : 0.0f;
    }
  };

  // The 8 waves' partial tiles summed through LDS in wave order, then the
  // epilogue (RoPE, GELU, LayerScale residual).
  auto reduce_and_store = [&](floatx4 (&acc)[NT]) {
    if (STAGE) __syncthreads();  // all waves are done with As before it becomes `red`
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) red[(wave * BM + 4 * g + r) * PR + 16 * j + li] = acc[j][r];
    __syncthreads();
    // OPT consecutive outputs per thread, BN / OPT threads per row.
    float out[OPT];
#pragma unroll
    for (int c = 0; c < OPT; ++c) {
      float v = red[er * PR + ec + c];
#pragma unroll
      for (int q = 1; q < NWV; ++q) v = __fadd_rn(v, red[(q * BM + er) * PR + ec + c]);
      out[c] = v;
    }
    if (rope || UPS) {
      __syncthreads();
#pragma unroll
      for (int c = 0; c < OPT; ++c) red[er * PR + ec + c] = out[c];
      __syncthreads();
    }
    if constexpr (UPS) {
      // Row er >= 1 is frame t = m; its two output rows read frames t and t - 1.
      if (er == 0 || m >= rows) return;
      const bool first = m % rows_per_seq == 0;
#pragma unroll
      for (int c = 0; c < OPT; ++c) {
        const int n = n0 + ec + c;
        const float cur = out[c], prev = red[(er - 1) * PR + ec + c];
#pragma unroll
        for (int q = 0; q < 2; ++q) {
          const float v = __fmul_rn(cur, up_w[n * 4 + q]);
          y[(2 * m + q) * N + n] = first ? v : __fadd_rn(__fmul_rn(prev, up_w[n * 4 + q + 2]), v);
        }
      }
      return;
    }
    if (m >= rows) return;
#pragma unroll
    for (int c = 0; c < OPT; ++c) {
      float v = out[c];
      if (rope) {
        const int d = ec + c;
        const float partner = red[er * PR + (d < 32 ? d + 32 : d - 32)];
        const float rot = d < 32 ? -partner : partner;
        v = __fadd_rn(__fmul_rn(v, e_cos[c]), __fmul_rn(rot, e_sin[c]));
      }
      if (flags & FM_EPI_GELU) v = fm_gelu(v);
      if (res_scale) v = __fadd_rn(e_res[c], __fmul_rn(e_scale[c], v));
      out[c] = v;
    }
    float* dst = y + m * N + n0 + ec;
    if constexpr (OPT == 2) {
      *reinterpret_cast<float2*>(dst) = float2{out[0], out[1]};
    } else {
#pragma unroll
      for (int c = 0; c < OPT; ++c) dst[c] = out[c];
    }
  };

  floatx4 acc[NT];
#pragma unroll
  for (int j = 0; j < NT; ++j) acc[j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  if constexpr (X6) {
    constexpr int KS = KW / 32, NU = 3 * KS;  // units: (k step, weight plane)
    // Weight units in flight: a ring of R (all of K = 512 at 32-column tiles,
    // four units of the 64-column tiles, six of the streamed K = 2048).
    constexpr int R0 = NT == 4 ? 4 : 6, R = R0 < NU ? R0 : NU;
    const __bf16* w3 = reinterpret_cast<const __bf16*>(wp);
    const long PL = (long)N * K;  // elements per plane
    // B fragment of k step st, tile j, plane pl: W rows n0 + 16 j + li, k = kw0 + 32 st + 8 g .. + 7,
    // i.e. k16-tile kw0 / 16 + 2 st + g / 2 at offset 8 (g & 1).
    const __bf16* wb3 = w3 + ((long)((kw0 >> 4) + (g >> 1)) * N + n0 + li) * 16 + 8 * (g & 1);
    const float* xs3 = x + min(m0 + li, (long)rows - 1) * K + kw0 + 8 * g;
    bf16x8 bu[R][NT];
    // A steps in flight: one ahead from LDS, three ahead when streamed from global memory.
    constexpr int RA0 = STAGE ? 2 : 4, RA = RA0 < KS ? RA0 : KS;
    floatx4 a3[RA][2];
    auto load_unit = [&](int buf, int u) {
      const int st = u / 3, pl = u % 3;
#pragma unroll
      for (int j = 0; j < NT; ++j)
        bu[buf][j] = *reinterpret_cast<const bf16x8*>(wb3 + pl * PL + (long)st * 2 * N * 16 + j * 256);
    };
    auto load_a3 = [&](int buf, int st) {
#pragma unroll
      for (int h = 0; h < 2; ++h)
        a3[buf][h] = STAGE ? *reinterpret_cast<const floatx4*>(As + li * PA + kw0 + 32 * st + 8 * g + 4 * h)
                           : *reinterpret_cast<const floatx4*>(xs3 + 32 * st + 4 * h);
    };
    auto load_ring = [&]() {
#pragma unroll
      for (int u = 0; u + 1 < R; ++u) load_unit(u, u);
    };
    if (!STAGE) load_ring();
    if (STAGE) {
      stage_rows();
      load_ring();
      __syncthreads();
    }
#pragma unroll
    for (int st = 0; st + 1 < RA; ++st) load_a3(st, st);
    if (RA == 1) load_a3(0, 0);
    fetch_epilogue();
    __builtin_amdgcn_sched_barrier(0);
    bf16x8 p0, p1, p2;
#pragma unroll
    for (int u = 0; u < NU; ++u) {
      const int st = u / 3, pl = u % 3, c = u % R;
      if (u + R - 1 < NU) load_unit((u + R - 1) % R, u + R - 1);
      if (pl == 0) {
        if (RA > 1 && st + RA - 1 < KS) load_a3((st + RA - 1) % RA, st + RA - 1);
        bf16x4 l0, l1, l2, h0, h1, h2;
        split3(a3[st % RA][0], l0, l1, l2);
        split3(a3[st % RA][1], h0, h1, h2);
        p0 = __builtin_shufflevector(l0, h0, 0, 1, 2, 3, 4, 5, 6, 7);
        p1 = __builtin_shufflevector(l1, h1, 0, 1, 2, 3, 4, 5, 6, 7);
        p2 = __builtin_shufflevector(l2, h2, 0, 1, 2, 3, 4, 5, 6, 7);
      }
      __builtin_amdgcn_sched_barrier(0);
      // Plane 0 of W meets all three A pieces, plane 1 the first two, plane 2
      // the first (the six terms of order <= 2); tiles interleaved.
      if (pl == 0) {
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j] = fm_mfma16_bf16(p2, bu[c][j], acc[j]);
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j] = fm_mfma16_bf16(p1, bu[c][j], acc[j]);
      } else if (pl == 1) {
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j] = fm_mfma16_bf16(p1, bu[c][j], acc[j]);
      }
#pragma unroll
      for (int j = 0; j < NT; ++j) acc[j] = fm_mfma16_bf16(p0, bu[c][j], acc[j]);
    }
    reduce_and_store(acc);
    return;
  }

  const long tstride = (long)(K / 64) * 4 * 64 * 4;  // floats between 16-column tiles
  const float* wb = wp + ((((long)(n0 / 16) * (K / 64) + kw0 / 64) * 4) * 64 + lane) * 4;
  const float* xs = x + min(m0 + li, (long)rows - 1) * K + kw0 + 16 * g;
  floatx4 a[2][4], b[2][NT][4];
  auto load_b = [&](int buf, int piece) {
#pragma unroll
    for (int j = 0; j < NT; ++j)
#pragma unroll
      for (int t = 0; t < 4; ++t)
        b[buf][j][t] = *reinterpret_cast<const floatx4*>(wb + j * tstride + piece * 1024 + t * 256);
  };
  auto load_a = [&](int buf, int piece) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      a[buf][t] = STAGE ? *reinterpret_cast<const floatx4*>(As + li * PA + kw0 + 64 * piece + 16 * g + 4 * t)
                        : *reinterpret_cast<const floatx4*>(xs + 64 * piece + 4 * t);
  };

  // The input rows are the critical path (LayerNorm, then the A operand).
  // With staging, the weight fragments are issued once the rows are in LDS:
  // issued earlier they queue ahead of the LayerNorm parameters and the
  // other waves' rows (measured 0.2-0.6 us faster per launch at 250 rows).
  if (!STAGE) load_b(0, 0);
  if (STAGE) {
    stage_rows();
    load_b(0, 0);
    __syncthreads();
  }
  load_a(0, 0);
  fetch_epilogue();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int pc = 0; pc < NP; ++pc) {
    const int c = pc & 1;
    if (pc + 1 < NP) {
      load_b(c ^ 1, pc + 1);
      load_a(c ^ 1, pc + 1);
    }
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t)
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int j = 0; j < NT; ++j) acc[j] = fm_mfma16(a[c][t][e], b[c][j][t][e], acc[j]);
  }
  reduce_and_store(acc);
}

// Packs W^T [N][K] (row-major) into the fragment order of row16_linear_kernel.
__global__ __launch_bounds__(256) void pack_row_weights_kernel(const float* __restrict__ w, int N,
                                                               int K, float* __restrict__ out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // float4 index in the packed array
  if (i >= (long)N * K / 4) return;
  const int lane = (int)(i % 64);
  const long q = i / 64;
  const int t = (int)(q % 4);
  const long q2 = q / 4;
  const int kp = (int)(q2 % (K / 64));
  const int nt = (int)(q2 / (K / 64));
  const int n = 16 * nt + lane % 16, k = 64 * kp + 16 * (lane / 16) + 4 * t;
  *reinterpret_cast<floatx4*>(out + 4 * i) = *reinterpret_cast<const floatx4*>(w + (long)n * K + k);
}


// In-place RoPE on the first rope_cols columns of each row (heads of
// head_dim, position = row % rows_per_seq into [*, head_dim] tables):
// x_d' = x_d*cos_d + rotate_half(x)_d*sin_d, products and sum rounded
// separately.  One thread per (row, head, d < head_dim / 2) pair.
__global__ __launch_bounds__(256) void apply_rope_kernel(float* x, long rows, int ld, int rope_cols,
                                                         int D, const float* __restrict__ cos_t,
                                                         const float* __restrict__ sin_t,
                                                         int rows_per_seq) {
  const int half = D / 2;
  const int pairs = rope_cols / 2;
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i >= rows * pairs) return;
  const long m = i / pairs;
  const int p = (int)(i % pairs);
  const int head = p / half, d = p % half;
  const long t = m % rows_per_seq;
  float* row = x + m * ld + head * D;
  const float lo = row[d], hi = row[d + half];
  row[d] = __fadd_rn(__fmul_rn(lo, cos_t[t * D + d]), __fmul_rn(-hi, sin_t[t * D + d]));
  row[d + half] = __fadd_rn(__fmul_rn(hi, cos_t[t * D + d + half]), __fmul_rn(lo, sin_t[t * D + d + half]));
}

}  // namespace

extern "C" {

// Transformer projection with optional fused LayerNorm prologue (gamma/beta
// non-null), RoPE epilogue on columns < rope_cols (cos/sin non-null; head_dim
// 64, tables [rows_per_seq][64]), GELU or LayerScale-residual epilogue.
// in_features must be 512 (Mimi's hidden width); out_features a multiple of 64.
int fm_row_linear_supported(int in_features, int out_features) {
  return (in_features == 512 || in_features == 2048) && out_features % 64 == 0;
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
  if (flags & FM_WEIGHTS_X6) {
    // bf16x6 planes after W^T: 16-row blocks on the bf16 matrix cores.
    if ((rows + 15) / 16 > 65535) return FM_UNSUPPORTED;
    if (in_features == 2048 && (ln_gamma || rope_cos)) return FM_UNSUPPORTED;
    const float* planes = weight + (long)out_features * in_features;
    const dim3 g64(out_features / 64, (rows + 15) / 16), g32(out_features / 32, (rows + 15) / 16);
    const bool wide = rope_cos || (long)(out_features / 32) * ((rows + 15) / 16) > 512;
#define FM_R16X6(KK, BN, G)                                                                           \
  hipLaunchKernelGGL((row16_linear_kernel<KK, BN, true>), G, dim3(512), 0, stream, x, rows, ln_gamma, \
                     ln_beta, ln_eps, planes, out_features, flags, residual, scale, rope_cos,        \
                     rope_sin, rope_cols, rows_per_seq, y)
    if (in_features == 2048) FM_R16X6(2048, 32, g32);
    else if (wide) FM_R16X6(512, 64, g64);
    else FM_R16X6(512, 32, g32);
#undef FM_R16X6
    return (int)hipGetLastError();
  }
  if ((rows + 31) / 32 > 65535) return FM_UNSUPPORTED;  // row blocks ride in grid y
  if (in_features == 2048) {  // streamed A operand: no LayerNorm / RoPE on this path
    if (ln_gamma || rope_cos) return FM_UNSUPPORTED;
    hipLaunchKernelGGL(row_stream_linear_kernel<2048>, dim3(out_features / 32, (rows + 31) / 32),
                       dim3(512), 0, stream, x, rows, weight, out_features, flags, residual, scale, y);
    return (int)hipGetLastError();
  }
  constexpr int K = 512;
  // 64-wide column tiles where RoPE needs whole heads, else 32-wide tiles (twice the blocks,
  // half the MFMA chain per wave); 8 waves split K.
  const bool wide = rope_cos != nullptr;
#define FM_ROWLIN(BN, NWV)                                                                       \
  {                                                                                              \
    const size_t lds = std::max<size_t>((size_t)32 * (K + 4), (size_t)NWV * 32 * (BN + 8)) * 4;  \
    hipLaunchKernelGGL((row_linear_kernel<K, BN, NWV>), dim3(out_features / BN, (rows + 31) / 32), \
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

// Few-row projections on fragment-packed weights (see row16_linear_kernel).
// Same arguments and epilogues as fm_row_linear; weight_packed comes from
// fm_pack_row_weights.  in_features 512 (LayerNorm / RoPE allowed) or 2048.
int fm_row_linear_packed(const float* x, int rows, int in_features, const float* ln_gamma,
                         const float* ln_beta, float ln_eps, const float* weight_packed,
                         int out_features, int flags, const float* residual, const float* scale,
                         const float* rope_cos, const float* rope_sin, int rope_cols,
                         int rows_per_seq, float* y, hipStream_t stream) {
  if (!x || !weight_packed || !y || rows < 0 || rows_per_seq <= 0 || (ln_gamma && !ln_beta))
    return FM_BAD_ARGUMENT;
  if (!fm_row_linear_supported(in_features, out_features)) return FM_UNSUPPORTED;
  if ((flags & FM_EPI_RES_SCALE) && (!residual || !scale)) return FM_BAD_ARGUMENT;
  if (rope_cos && (!rope_sin || rope_cols % 64)) return FM_BAD_ARGUMENT;
  if (rows == 0) return FM_OK;
  if ((rows + 15) / 16 > 65535) return FM_UNSUPPORTED;  // row blocks ride in grid y
  if (in_features == 2048 && (ln_gamma || rope_cos)) return FM_UNSUPPORTED;
  const dim3 g64(out_features / 64, (rows + 15) / 16), g32(out_features / 32, (rows + 15) / 16);
#define FM_R16(KK, BN, G)                                                                       \
  hipLaunchKernelGGL((row16_linear_kernel<KK, BN>), G, dim3(512), 0, stream, x, rows, ln_gamma, \
                     ln_beta, ln_eps, weight_packed, out_features, flags, residual, scale,     \
                     rope_cos, rope_sin, rope_cols, rows_per_seq, y)
  // 64-column blocks where RoPE needs whole heads, or where 32-column blocks
  // would not all be resident at once (two 8-wave blocks per CU).
  const bool wide = rope_cos || (long)(out_features / 32) * ((rows + 15) / 16) > 512;
  if (in_features == 2048) FM_R16(2048, 32, g32);
  else if (wide) FM_R16(512, 64, g64);
  else FM_R16(512, 32, g32);
#undef FM_R16
  return (int)hipGetLastError();
}

// Projection of the RVQ decoder output followed by the bottleneck's
// depthwise ConvTranspose1d upsample (kernel 4, stride 2), in one launch.
int fm_row_linear_packed_upsample(const float* x, int rows, int in_features,
                                  const float* weight_packed, int out_features, int rows_per_seq,
                                  const float* up_weight, float* y, hipStream_t stream) {
  if (!x || !weight_packed || !up_weight || !y || rows < 0 || rows_per_seq <= 0)
    return FM_BAD_ARGUMENT;
  if (in_features != 512 || out_features <= 0 || out_features % 32) return FM_UNSUPPORTED;
  if (rows == 0) return FM_OK;
  const long blocks = (rows + 14) / 15;  // 15 new frames per 16-row block
  if (blocks > 65535) return FM_UNSUPPORTED;
  hipLaunchKernelGGL((row16_linear_kernel<512, 32, false, true>), dim3(out_features / 32, (unsigned)blocks),
                     dim3(512), 0, stream, x, rows, nullptr, nullptr, 0.0f, weight_packed, out_features, 0,
                     nullptr, nullptr, nullptr, nullptr, 0, rows_per_seq, y, up_weight);
  return (int)hipGetLastError();
}

// Packs a [out_features][in_features] weight for fm_row_linear_packed
// (out_features % 16 == 0, in_features % 64 == 0).  out must not alias weight.
int fm_pack_row_weights(const float* weight, int out_features, int in_features, float* out,
                        hipStream_t stream) {
  if (!weight || !out || out_features <= 0 || in_features <= 0 || out_features % 16 ||
      in_features % 64 || weight == out)
    return FM_BAD_ARGUMENT;
  const long n4 = (long)out_features * in_features / 4;
  hipLaunchKernelGGL(pack_row_weights_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0,
                     stream, weight, out_features, in_features, out);
  return (int)hipGetLastError();
}

// In-place RoPE for projections made without the fused epilogue.
int fm_apply_rope(float* x, long rows, int ld, int rope_cols, int head_dim, const float* cos_table,
                  const float* sin_table, int rows_per_seq, hipStream_t stream) {
  if (!x || !cos_table || !sin_table || rows < 0 || head_dim <= 0 || head_dim % 2 ||
      rope_cols % head_dim || rope_cols > ld || rows_per_seq <= 0)
    return FM_BAD_ARGUMENT;
  const long total = rows * (rope_cols / 2);
  if (total == 0) return FM_OK;
  hipLaunchKernelGGL(apply_rope_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, stream,
                     x, rows, ld, rope_cols, head_dim, cos_table, sin_table, rows_per_seq);
  return (int)hipGetLastError();
}

int fm_layer_norm(const float* x, const float* gamma, const float* beta, long rows, int channels,
                  float eps, float* y, hipStream_t stream) {
  if (!x || !gamma || !beta || !y || rows < 0 || channels <= 0) return FM_BAD_ARGUMENT;
  if (rows == 0) return FM_OK;
  const long blocks = (rows + 3) / 4;
  if (channels == 512 && ((uintptr_t)x | (uintptr_t)y | (uintptr_t)gamma | (uintptr_t)beta) % 16 == 0) {
    hipLaunchKernelGGL(layer_norm512_kernel, dim3((unsigned)((rows + 7) / 8)), dim3(256), 0, stream,
                       x, gamma, beta, rows, eps, y);
    return (int)hipGetLastError();
  }
  hipLaunchKernelGGL(layer_norm_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, x, gamma,
                     beta, rows, channels, eps, y);
  return (int)hipGetLastError();
}

int fm_window_attention_rows(const float* qkv, int ld_qkv, int q_offset, int k_offset,
                             int v_offset, const float* cos_table, const float* sin_table,
                             int batch, int length, int query_start, int heads, int kv_heads,
                             int head_dim, int window, float scale, float* out, int ld_out,
                             hipStream_t stream);

int fm_window_attention(const float* qkv, int ld_qkv, int q_offset, int k_offset, int v_offset,
                        const float* cos_table, const float* sin_table, int batch, int length,
                        int heads, int kv_heads, int head_dim, int window, float scale, float* out,
                        int ld_out, hipStream_t stream) {
  return fm_window_attention_rows(qkv, ld_qkv, q_offset, k_offset, v_offset, cos_table, sin_table,
                                  batch, length, 0, heads, kv_heads, head_dim, window, scale, out,
                                  ld_out, stream);
}

// Attention for the queries at rows query_start .. length-1 of each sequence;
// every row 0 .. length-1 is a key/value (rows before query_start hold a KV
// cache).  out has length - query_start rows per sequence.
int fm_window_attention_rows(const float* qkv, int ld_qkv, int q_offset, int k_offset,
                             int v_offset, const float* cos_table, const float* sin_table,
                             int batch, int length, int query_start, int heads, int kv_heads,
                             int head_dim, int window, float scale, float* out, int ld_out,
                             hipStream_t stream) {
  if (!qkv || !cos_table != !sin_table || !out || batch < 0 || length < 0 || heads <= 0 ||
      kv_heads <= 0 || heads % kv_heads || window <= 0)
    return FM_BAD_ARGUMENT;
  // Q/K/V rows are read as float4s.
  if ((ld_qkv | q_offset | k_offset | v_offset) % 4) return FM_BAD_ARGUMENT;
  if (query_start < 0 || query_start > length) return FM_BAD_ARGUMENT;
  if (batch == 0 || length == query_start) return FM_OK;
  if (head_dim == 64 && query_start == 0 && length <= SEQ_MAX && (long)batch * heads >= 128) {
    // Enough (sequence, head) pairs to fill the GPU with two blocks each.
    const dim3 gs(2, heads, batch);
    constexpr int NKS = 2;
    if (cos_table)
      hipLaunchKernelGGL((window_attention_seq_kernel<true, NKS>), gs, dim3(256 * NKS), 0, stream, qkv,
                         ld_qkv, q_offset, k_offset, v_offset, cos_table, sin_table, length, heads,
                         kv_heads, window, scale, out, ld_out);
    else
      hipLaunchKernelGGL((window_attention_seq_kernel<false, NKS>), gs, dim3(256 * NKS), 0, stream, qkv,
                         ld_qkv, q_offset, k_offset, v_offset, cos_table, sin_table, length, heads,
                         kv_heads, window, scale, out, ld_out);
    return (int)hipGetLastError();
  }
  if (head_dim == 64 && length - query_start >= 512 && (long)batch * heads < 128) {
    // Long sequences, few sequence-heads: query blocks sharing each key chunk.
    constexpr int NWQ = 2;
    const dim3 gf((length - query_start + 16 * NWQ - 1) / (16 * NWQ), heads, batch);
    if (cos_table)
      hipLaunchKernelGGL((window_attention_flash_kernel<true, NWQ>), gf, dim3(64 * NWQ), 0, stream, qkv, ld_qkv,
                         q_offset, k_offset, v_offset, cos_table, sin_table, length, query_start,
                         heads, kv_heads, window, scale, out, ld_out);
    else
      hipLaunchKernelGGL((window_attention_flash_kernel<false, NWQ>), gf, dim3(64 * NWQ), 0, stream, qkv, ld_qkv,
                         q_offset, k_offset, v_offset, cos_table, sin_table, length, query_start,
                         heads, kv_heads, window, scale, out, ld_out);
    return (int)hipGetLastError();
  }
  if (head_dim == 64) {
    // 16-query blocks; eight waves per block (fewer key tiles per wave) while
    // the grid is too small to fill the GPU, four once blocks are plentiful.
    const dim3 g16((length - query_start + 15) / 16, heads, batch);
    const bool eight16 = (long)g16.x * g16.y * g16.z < 1024;
#define FM_ATT16(R, W)                                                                             hipLaunchKernelGGL((window_attention16_kernel<R, W>), g16, dim3(64 * W), 0, stream, qkv, ld_qkv,                      q_offset, k_offset, v_offset, cos_table, sin_table, length, query_start,                           heads, kv_heads, window, scale, out, ld_out)
    if (cos_table) {
      if (eight16) FM_ATT16(true, 8);
      else FM_ATT16(true, 4);
    } else {
      if (eight16) FM_ATT16(false, 8);
      else FM_ATT16(false, 4);
    }
#undef FM_ATT16
    return (int)hipGetLastError();
  }
  dim3 grid((length - query_start + QB - 1) / QB, heads, batch);
  // Eight waves per block (fewer key tiles per wave) while the grid is too
  // small to fill the GPU; four once blocks are plentiful.
  const bool eight = (long)grid.x * grid.y * grid.z < 512;
#define FM_ATT_NW(DV, R, W)                                                                  \
  hipLaunchKernelGGL((window_attention_kernel<DV, R, W>), grid, dim3(64 * W), 0, stream, qkv, \
                     ld_qkv, q_offset, k_offset, v_offset, cos_table, sin_table, length,      \
                     query_start, heads, kv_heads, window, scale, out, ld_out)
#define FM_ATT(DV)                                  \
  if (cos_table) {                                  \
    if (eight) FM_ATT_NW(DV, true, 8);              \
    else FM_ATT_NW(DV, true, 4);                    \
  } else {                                          \
    if (eight) FM_ATT_NW(DV, false, 8);             \
    else FM_ATT_NW(DV, false, 4);                   \
  }
  switch (head_dim) {
    case 8: FM_ATT(8); break;
    case 16: FM_ATT(16); break;
    case 32: FM_ATT(32); break;
    default: return FM_UNSUPPORTED;
  }
#undef FM_ATT
#undef FM_ATT_NW
  return (int)hipGetLastError();
}

}  // extern "C"
