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

constexpr int QB = 32;  // queries per block
constexpr int KC = 64;  // keys per staged chunk

// RoPE as the reference writes it: x*cos + rotate_half(x)*sin, no contraction.
FM_DEVICE float rope(const float* v, int d, int D, const float* cs, const float* sn) {
  const int h = D / 2;
  const float rot = d < h ? -v[d + h] : v[d - h];
  return __fadd_rn(__fmul_rn(v[d], cs[d]), __fmul_rn(rot, sn[d]));
}

// Grid: (ceil(T / QB), heads, batch); 256 threads = 8 threads per query.
template <int D>
__global__ __launch_bounds__(256) void window_attention_kernel(
    const float* __restrict__ qkv, int ld, int q_off, int k_off, int v_off,
    const float* __restrict__ cos_t, const float* __restrict__ sin_t, int T, int heads,
    int kv_heads, int window, float scale, float* __restrict__ out, int ld_out) {
  constexpr int P = D + 1;
  __shared__ float Qs[QB * P];
  __shared__ float Ks[KC * P];
  __shared__ float Vs[KC * P];
  __shared__ float Ps[QB * (KC + 1)];

  const int tid = threadIdx.x;
  const int qi = tid >> 3;   // query within block
  const int sub = tid & 7;   // lane within the query's group of 8
  const int h = blockIdx.y;
  const int hk = h / (heads / kv_heads);
  const long b = blockIdx.z;
  const int q0 = blockIdx.x * QB;
  const int qlast = min(q0 + QB, T) - 1;
  const int k_lo = max(0, q0 - window + 1);
  const int k_hi = qlast;
  const long base = b * (long)T;

  // Stage Q with RoPE.
  for (int e = tid; e < QB * D; e += 256) {
    const int r = e / D, d = e % D;
    const int t = q0 + r;
    float v = 0.0f;
    if (t < T) {
      const float* src = qkv + (base + t) * ld + q_off + h * D;
      v = rope(src, d, D, cos_t + (long)t * D, sin_t + (long)t * D);
    }
    Qs[r * P + d] = v;
  }

  const int qg = q0 + qi;
  float m_run = -INFINITY, l_run = 0.0f;
  float o[D / 8];
#pragma unroll
  for (int i = 0; i < D / 8; ++i) o[i] = 0.0f;

  for (int k0 = k_lo; k0 <= k_hi; k0 += KC) {
    __syncthreads();
    for (int e = tid; e < KC * D; e += 256) {
      const int r = e / D, d = e % D;
      const int t = k0 + r;
      float kv = 0.0f, vv = 0.0f;
      if (t <= k_hi) {
        const float* row = qkv + (base + t) * ld;
        kv = rope(row + k_off + hk * D, d, D, cos_t + (long)t * D, sin_t + (long)t * D);
        vv = row[v_off + hk * D + d];
      }
      Ks[r * P + d] = kv;
      Vs[r * P + d] = vv;
    }
    __syncthreads();

    float s[KC / 8];
    float cmax = -INFINITY;
#pragma unroll
    for (int i = 0; i < KC / 8; ++i) {
      const int kk = sub + 8 * i;
      const int kg = k0 + kk;
      float acc = 0.0f;
#pragma unroll 16
      for (int d = 0; d < D; ++d) acc = fmaf(Qs[qi * P + d], Ks[kk * P + d], acc);
      const bool ok = qg < T && kg <= k_hi && kg <= qg && kg > qg - window;
      s[i] = ok ? acc * scale : -INFINITY;
      cmax = fmaxf(cmax, s[i]);
    }
#pragma unroll
    for (int o2 = 1; o2 < 8; o2 <<= 1) cmax = fmaxf(cmax, __shfl_xor(cmax, o2, 64));
    const float m_new = fmaxf(m_run, cmax);
    float psum = 0.0f;
#pragma unroll
    for (int i = 0; i < KC / 8; ++i) {
      const float pv = (m_new == -INFINITY || s[i] == -INFINITY) ? 0.0f : expf(s[i] - m_new);
      Ps[qi * (KC + 1) + sub + 8 * i] = pv;
      psum += pv;
    }
#pragma unroll
    for (int o2 = 1; o2 < 8; o2 <<= 1) psum += __shfl_xor(psum, o2, 64);
    const float corr = (m_run == -INFINITY) ? 0.0f : expf(m_run - m_new);
    l_run = l_run * corr + psum;
    m_run = m_new;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < D / 8; ++i) {
      const int d = sub + 8 * i;
      float acc = o[i] * corr;
      for (int kk = 0; kk < KC; ++kk) acc = fmaf(Ps[qi * (KC + 1) + kk], Vs[kk * P + d], acc);
      o[i] = acc;
    }
  }
  if (qg < T) {
    float* dst = out + (base + qg) * ld_out + h * D;
    const float inv = 1.0f / l_run;
#pragma unroll
    for (int i = 0; i < D / 8; ++i) dst[sub + 8 * i] = o[i] * inv;
  }
}

}  // namespace

extern "C" {

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
  if (!qkv || !cos_table || !sin_table || !out || batch < 0 || length < 0 || heads <= 0 ||
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
