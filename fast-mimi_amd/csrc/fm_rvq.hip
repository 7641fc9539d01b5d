// Split residual vector quantizer of the Mimi hot path.
//
// Encode, one launch per codebook step j (the residual chain is sequential):
//   each block owns RB query rows and one chunk of codebook entries;
//   prologue (j > 0): resolve step j-1's argmin from its per-chunk partials,
//     residual_j = residual_{j-1} - e_{j-1}[code]  (one FP32 subtract, as the
//     reference's ``residual - quantized``), chunk-0 blocks publish the
//     residual and step j-1's code;
//   main: distance GEMM on FP32 MFMA against the transposed codebook,
//     d = (-2 x.e + |x|^2) + |e|^2 -> clamp(0) -> sqrt (torch cdist's mm form),
//     and a lowest-index argmin reduced across lanes and waves.
// A finalize launch resolves the last step.
//
// Decode: ordered gather-sum (0 + e_0[c_0] for the semantic branch,
// 0 + e_1[c_1] + e_2[c_2] + ... left to right for the acoustic branch) into
// the [rows, 2*dim] operand of the fused output projection GEMM.

#include <cstdlib>

#include "fm_common.h"

namespace {

constexpr int RB = 32;  // query rows per block
constexpr int kQt2MaxChunkEntries = 2048;  // codebook entries per block with 64-row blocks
constexpr int kMaxChunks = 64;  // entry chunks per step (partials per row)

FM_DEVICE bool better(float v, int i, float bv, int bi) {
  return v < bv || (v == bv && i < bi);
}

// cdist value of one mm-form distance as an argmin key.  torch's clamp_min
// keeps a NaN and its argmin returns the first NaN, so a NaN maps to -inf:
// it then beats every real distance (all >= 0) and ties between NaNs go to
// the lowest index.  Non-finite input rows therefore still yield a valid code.
FM_DEVICE float dist_key(float d) {
  return d != d ? -INFINITY : sqrtf(fmaxf(d, 0.0f));
}

// A resolved code used as a gather index.  Every resolve visits at least one
// entry, so the index is in range; the clamp keeps a gather inside the
// codebook whatever the partials hold.
FM_DEVICE int code_index(int code, int entries) {
  return (unsigned)code < (unsigned)entries ? code : 0;
}

struct StepArgs {
  const float* resid_in;   // rows entering step j-1 (or step 0), row pitch ld_in
  int ld_in;
  const float* prev_embed; // codebook j-1 [entries][dim]; null at step 0
  const float* prev_val;   // step j-1 partials [chunks][M]
  const int* prev_idx;
  float* resid_out;        // residual_j [M][dim] (chunk-0 blocks write it); may be null at step 0
  int64_t* prev_codes;     // codes of step j-1 (row (b,t) at b*batch_stride + t)
  const float* embed_t;    // codebook j transposed [dim][entries]
  const float* norms;      // |e|^2 [entries]
  float* val;              // step j partials [chunks][M]
  int* idx;
  int M, dim, entries, chunk_entries, chunks, rows_per_batch, batch_stride;
};

FM_DEVICE void resolve(const float* val, const int* idx, int chunks, long M, long m, float& bv,
                       int& bi) {
  bv = val[m];
  bi = idx[m];
  for (int c = 1; c < chunks; ++c) {
    const float v = val[(long)c * M + m];
    const int i = idx[(long)c * M + m];
    if (better(v, i, bv, bi)) bv = v, bi = i;
  }
}

// Argmin over the chunk partials of row m, spread over the 8 lanes pt = 0..7
// of an aligned lane group: lane pt takes chunks pt, pt + 8, ... (at most
// kMaxChunks / 8), all loads issued before the first compare, then the 8
// lanes are shuffle-reduced.  ``better`` is a total order, so the result is
// the lowest-index minimum whatever the reduction order.
FM_DEVICE void resolve8(const float* val, const int* idx, int chunks, long M, long m, int pt,
                        float& bv, int& bi) {
  constexpr int PER = kMaxChunks / 8;
  float v[PER];
  int ix[PER];
#pragma unroll
  for (int u = 0; u < PER; ++u) {
    const int c = pt + 8 * u;
    const int cc = min(c, chunks - 1);
    v[u] = val[(long)cc * M + m];
    ix[u] = idx[(long)cc * M + m];
    if (c >= chunks) v[u] = INFINITY, ix[u] = 0x7fffffff;
  }
  bv = v[0];
  bi = ix[0];
#pragma unroll
  for (int u = 1; u < PER; ++u)
    if (better(v[u], ix[u], bv, bi)) bv = v[u], bi = ix[u];
#pragma unroll
  for (int o = 1; o < 8; o <<= 1) {
    const float ov = __shfl_xor(bv, o, 64);
    const int oi = __shfl_xor(bi, o, 64);
    if (better(ov, oi, bv, bi)) bv = ov, bi = oi;
  }
}

constexpr int NT = 128;  // entries per sub-tile (4 waves x 32)
constexpr int KSL = 32;  // codebook dims per staged slice
constexpr int PB = NT + 4;

// Dynamic LDS: Xs[dim][RB+1] (k-major, MFMA A operand), Bs[KSL][NT+4]
// (staged codebook slice), xn[RB], per-wave best (value, index), codes[RB].
__global__ __launch_bounds__(256) void rvq_step_kernel(StepArgs a) {
  extern __shared__ float smem[];
  constexpr int PX = RB + 1;
  float* Xs = smem;
  float* Bs = Xs + a.dim * PX;
  float* xn = Bs + KSL * PB;
  float* bval = xn + RB;
  int* bidx = reinterpret_cast<int*>(bval + 4 * RB);
  int* rcode = bidx + 4 * RB;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const long m0 = (long)blockIdx.x * RB;
  const int chunk = blockIdx.y;

  if (a.prev_embed && tid < RB) {
    const long m = m0 + tid;
    int code = 0;
    if (m < a.M) {
      float bv;
      resolve(a.prev_val, a.prev_idx, a.chunks, a.M, m, bv, code);
      code = code_index(code, a.entries);
      if (chunk == 0) {
        const long b = m / a.rows_per_batch, t = m - b * a.rows_per_batch;
        a.prev_codes[b * a.batch_stride + t] = code;
      }
    }
    rcode[tid] = code;
  }
  __syncthreads();
  // Residual rows into LDS.  All loads of a batch are issued before any
  // store, so they overlap instead of queueing behind possibly-aliasing stores.
  {
    const int dv = a.dim / 4;  // dim is a multiple of 4 on this path
    const int total = RB * dv;
    constexpr int UNR = 8;
    for (int c0 = 0; c0 < total; c0 += 256 * UNR) {
      floatx4 xv[UNR], ev[UNR];
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int c = c0 + u * 256 + tid;
        const int r = c / dv, k = (c % dv) * 4;
        const long m = m0 + r;
        xv[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        ev[u] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
        if (c < total && m < a.M) {
          xv[u] = *reinterpret_cast<const floatx4*>(a.resid_in + m * a.ld_in + k);
          if (a.prev_embed)
            ev[u] = *reinterpret_cast<const floatx4*>(a.prev_embed + (long)rcode[r] * a.dim + k);
        }
      }
#pragma unroll
      for (int u = 0; u < UNR; ++u) {
        const int c = c0 + u * 256 + tid;
        if (c >= total) continue;
        const int r = c / dv, k = (c % dv) * 4;
        const long m = m0 + r;
        floatx4 x = xv[u];
        if (a.prev_embed && m < a.M) {
          x.x = __fsub_rn(x.x, ev[u].x);
          x.y = __fsub_rn(x.y, ev[u].y);
          x.z = __fsub_rn(x.z, ev[u].z);
          x.w = __fsub_rn(x.w, ev[u].w);
          if (chunk == 0 && a.resid_out) *reinterpret_cast<floatx4*>(a.resid_out + m * a.dim + k) = x;
        }
        Xs[(k + 0) * PX + r] = x.x;
        Xs[(k + 1) * PX + r] = x.y;
        Xs[(k + 2) * PX + r] = x.z;
        Xs[(k + 3) * PX + r] = x.w;
      }
    }
  }
  __syncthreads();
  if (tid < RB) {
    float s = 0.0f;
    for (int k = 0; k < a.dim; ++k) s = fmaf(Xs[k * PX + tid], Xs[k * PX + tid], s);
    xn[tid] = s;
  }

  float best_v[16];
  int best_i[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) best_v[r] = INFINITY, best_i[r] = 0x7fffffff;
  const int e_begin = chunk * a.chunk_entries;
  const int e_end = min(a.entries, e_begin + a.chunk_entries);
  const int lrow = lane >> 5, lcol = lane & 31;
  const bool vec = (a.entries % 4 == 0);
  for (int n0 = e_begin; n0 < e_end; n0 += NT) {
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
    for (int k0 = 0; k0 < a.dim; k0 += KSL) {
      __syncthreads();
      // Stage codebook dims [k0, k0+KSL) x entries [n0, n0+NT) (rows contiguous in entries).
      if (vec) {
        for (int c = tid; c < KSL * NT / 4; c += 256) {
          const int kr = c / (NT / 4), nn = (c % (NT / 4)) * 4;
          const int k = k0 + kr, n = n0 + nn;
          floatx4 v = {0.0f, 0.0f, 0.0f, 0.0f};
          if (k < a.dim && n < e_end) v = *reinterpret_cast<const floatx4*>(a.embed_t + (long)k * a.entries + n);
          *reinterpret_cast<floatx4*>(&Bs[kr * PB + nn]) = v;
        }
      } else {
        for (int c = tid; c < KSL * NT; c += 256) {
          const int kr = c / NT, nn = c % NT;
          const int k = k0 + kr, n = n0 + nn;
          Bs[kr * PB + nn] = (k < a.dim && n < e_end) ? a.embed_t[(long)k * a.entries + n] : 0.0f;
        }
      }
      __syncthreads();
      const int kmax = min(KSL, a.dim - k0);
#pragma unroll 8
      for (int kk = 0; kk < kmax; kk += 2) {
        const float av = Xs[(k0 + kk + lrow) * PX + lcol];
        const float bv = Bs[(kk + lrow) * PB + wave * 32 + lcol];
        acc = fm_mfma32(av, bv, acc);
      }
    }
    const int col = n0 + wave * 32 + lcol;
    if (col < e_end) {
      const float en = a.norms[col];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = fm_mfma32_row(r, lane);
        const float d = __fadd_rn(__fadd_rn(__fmul_rn(-2.0f, acc[r]), xn[row]), en);
        const float dist = dist_key(d);
        if (better(dist, col, best_v[r], best_i[r])) best_v[r] = dist, best_i[r] = col;
      }
    }
  }
  // Reduce across the 32 lanes that share each row.
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    float v = best_v[r];
    int i = best_i[r];
#pragma unroll
    for (int o = 1; o < 32; o <<= 1) {
      const float ov = __shfl_xor(v, o, 64);
      const int oi = __shfl_xor(i, o, 64);
      if (better(ov, oi, v, i)) v = ov, i = oi;
    }
    if (lcol == 0) {
      const int row = fm_mfma32_row(r, lane);
      bval[wave * RB + row] = v;
      bidx[wave * RB + row] = i;
    }
  }
  __syncthreads();
  if (tid < RB) {
    const long m = m0 + tid;
    float v = bval[tid];
    int i = bidx[tid];
    for (int w = 1; w < 4; ++w)
      if (better(bval[w * RB + tid], bidx[w * RB + tid], v, i)) v = bval[w * RB + tid], i = bidx[w * RB + tid];
    if (m < a.M) {
      a.val[(long)chunk * a.M + m] = v;
      a.idx[(long)chunk * a.M + m] = i;
    }
  }
}

// Fast step kernel for dim in {64, 128, 256}.  Block = RB query rows x one
// chunk of entries, 4 waves = EG entry groups x KP k-parts (KP * EG == 4).
// MFMA rows are codebook entries (A operand loaded straight from the
// row-major codebook into registers, one 64-dim piece ahead of its use),
// columns are queries (B operand from the LDS residual rows).  In a 64-dim
// piece the k-slot of lane half h at step 4j+e carries dim 32h + 4j + e, so
// both operands are 16-byte reads.  Each lane then holds the 16 candidate
// distances of its query for one 32-entry sub-tile, so the argmin is a
// register scan plus one cross-half shuffle.  With KP > 1 every wave owns one
// sub-tile and one k-part; partial dot products are summed through LDS in
// k-part order before the distances.  The prologue resolves step j-1 (eight
// lanes per row, shuffle-reduced) and forms residual_j and |residual_j|^2.
template <int DIM, int KP, int QTN = 1>
__global__ __launch_bounds__(256) void rvq_step_mfma_kernel(StepArgs a0, const float* __restrict__ e0,
                                                            StepArgs a1, const float* __restrict__ e1) {
  // QTN = 2: 64 query rows per block as two 32-query MFMA column tiles that
  // share every codebook fragment (half the codebook reads per query).
  static_assert(QTN == 1 || (QTN == 2 && KP == 1), "two query tiles only without k-parts");
  constexpr int RBT = RB * QTN;
  // blockIdx.z picks the branch (semantic / acoustic chains share launches).
  const StepArgs a = blockIdx.z ? a1 : a0;
  const float* __restrict__ embed = blockIdx.z ? e1 : e0;
  // A branch one step past its last codebook only resolves that codebook
  // (chunk-0 blocks write the codes).
  const bool fin = a.embed_t == nullptr;
  if (fin && blockIdx.y != 0) return;
  constexpr int EG = 4 / KP, KW = DIM / KP, NPC = KW / 64, PX = DIM + 4, PR = RB + 1;
  constexpr int CH = DIM / 32;  // float4 chunks per lane in the prologue (8 lanes per row)
  static_assert(KW % 64 == 0, "k-part of whole 64-dim pieces");
  // QTN = 2 needs more than the 64 KB of dynamic LDS a launch gets: a static
  // array sized for 64 rows and up to kQt2MaxChunkEntries codebook norms.
  extern __shared__ __attribute__((aligned(16))) float smem_dyn[];
  __shared__ __attribute__((aligned(16))) float smem_qt2[QTN == 2 ? RBT * PX + RBT + 2 * 4 * RBT + kQt2MaxChunkEntries : 4];
  float* smem = QTN == 2 ? smem_qt2 : smem_dyn;
  float* Xs = smem;                      // [RBT][PX]
  float* xnS = Xs + RBT * PX;            // [RBT]
  float* bestv = xnS + RBT;              // [EG][RBT]
  int* besti = reinterpret_cast<int*>(bestv + EG * RBT);
  float* red = reinterpret_cast<float*>(besti + EG * RBT);  // [KP-1][EG][32 * PR]
  float* normS = red + (KP - 1) * EG * 32 * PR;            // [chunk_entries]

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int g = wave % EG, p = wave / EG;
  const int h = lane >> 5, col = lane & 31;
  const long m0 = (long)blockIdx.x * RBT;
  const int chunk = blockIdx.y;
  const int e_begin = chunk * a.chunk_entries;
  const int e_end = min(a.entries, e_begin + a.chunk_entries);

  // The first codebook piece does not depend on the previous step: its
  // loads go out before the prologue's dependent chain.
  const int nsub = (e_end - e_begin + 31) / 32;
  const int my_sub = (nsub - g + EG - 1) / EG;  // sub-tiles g, g+EG, ...
  const int items = (KP == 1) ? my_sub * NPC : NPC;
  const int kbase = p * KW;
  floatx4 cur[8], nxt[8];
  auto load_piece = [&](floatx4* dst, int item) {
    const int st = g + EG * ((KP == 1) ? item / NPC : 0);
    const int pc = item % NPC;
    const int entry = min(e_begin + 32 * st + col, a.entries - 1);
    const float* src = embed + (long)entry * DIM + kbase + 64 * pc + 32 * h;
#pragma unroll
    for (int j = 0; j < 8; ++j) dst[j] = *reinterpret_cast<const floatx4*>(src + 4 * j);
  };
  const bool has_work = !fin && (KP == 1 ? items > 0 : g < nsub);
  if (has_work) load_piece(cur, 0);

  // ---- prologue: rows r = 32 * pass + tid / 8, lane part pt = tid % 8.
  {
    const int pt = tid & 7;
    // The residual rows do not depend on the previous code: issue them first.
    floatx4 xv[QTN][CH];
    if (!fin) {
#pragma unroll
      for (int ps = 0; ps < QTN; ++ps) {
        const long mc = min(m0 + 32 * ps + (tid >> 3), (long)a.M - 1);
#pragma unroll
        for (int u = 0; u < CH; ++u)
          xv[ps][u] = *reinterpret_cast<const floatx4*>(a.resid_in + mc * a.ld_in + 4 * (pt + 8 * u));
      }
    }
    int code[QTN];
#pragma unroll
    for (int ps = 0; ps < QTN; ++ps) {
      code[ps] = 0;
      const long m = m0 + 32 * ps + (tid >> 3);
      const long mc = min(m, (long)a.M - 1);
      if (a.prev_embed) {
        float bv;
        int bi;
        resolve8(a.prev_val, a.prev_idx, a.chunks, a.M, mc, pt, bv, bi);
        bi = code_index(bi, a.entries);
        code[ps] = bi;
        if (chunk == 0 && pt == 0 && m < a.M) {
          const long b = m / a.rows_per_batch, t = m - b * a.rows_per_batch;
          a.prev_codes[b * a.batch_stride + t] = bi;
        }
      }
    }
    if (fin) return;
    for (int c = tid; c < e_end - e_begin; c += 256) normS[c] = a.norms[e_begin + c];
#pragma unroll
    for (int ps = 0; ps < QTN; ++ps) {
      const int r = 32 * ps + (tid >> 3);
      const long m = m0 + r;
      const bool valid = m < a.M;
      floatx4 ev[CH];
      if (a.prev_embed) {
#pragma unroll
        for (int u = 0; u < CH; ++u)
          ev[u] = *reinterpret_cast<const floatx4*>(a.prev_embed + (long)code[ps] * DIM + 4 * (pt + 8 * u));
      }
      float xn = 0.0f;
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        floatx4 x = xv[ps][u];
        if (a.prev_embed) {
#pragma unroll
          for (int e = 0; e < 4; ++e) x[e] = __fsub_rn(x[e], ev[u][e]);
          if (chunk == 0 && valid && a.resid_out)
            *reinterpret_cast<floatx4*>(a.resid_out + m * DIM + 4 * (pt + 8 * u)) = x;
        }
        if (!valid) x = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 4; ++e) xn = fmaf(x[e], x[e], xn);
        *reinterpret_cast<floatx4*>(Xs + r * PX + 4 * (pt + 8 * u)) = x;
      }
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) xn += __shfl_xor(xn, o, 64);
      if (pt == 0) xnS[r] = xn;
    }
  }
  __syncthreads();

  // ---- distance tiles.
  float xq[QTN], best_vq[QTN];
  int best_iq[QTN];
  floatx16 accq[QTN];
#pragma unroll
  for (int qt = 0; qt < QTN; ++qt) {
    xq[qt] = xnS[col + 32 * qt];
    best_vq[qt] = INFINITY;
    best_iq[qt] = 0x7fffffff;
#pragma unroll
    for (int r = 0; r < 16; ++r) accq[qt][r] = 0.0f;
  }
  for (int it = 0; it < (has_work ? items : 0); ++it) {
    if (it + 1 < items) load_piece(nxt, it + 1);
    const int pc = it % NPC;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
#pragma unroll
      for (int qt = 0; qt < QTN; ++qt) {
        const floatx4 b4 =
            *reinterpret_cast<const floatx4*>(Xs + (col + 32 * qt) * PX + kbase + 64 * pc + 32 * h + 4 * j);
#pragma unroll
        for (int e = 0; e < 4; ++e) accq[qt] = fm_mfma32(cur[j][e], b4[e], accq[qt]);
      }
    }
#pragma unroll
    for (int j = 0; j < 8; ++j) cur[j] = nxt[j];
    if (KP == 1 && pc == NPC - 1) {
      const int n0 = e_begin + 32 * (g + EG * (it / NPC));
#pragma unroll
      for (int qt = 0; qt < QTN; ++qt)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int entry = n0 + fm_mfma32_row(r, lane);
          if (entry < e_end) {
            const float d = __fadd_rn(__fadd_rn(__fmul_rn(-2.0f, accq[qt][r]), xq[qt]), normS[entry - e_begin]);
            const float dist = dist_key(d);
            if (better(dist, entry, best_vq[qt], best_iq[qt])) best_vq[qt] = dist, best_iq[qt] = entry;
          }
          accq[qt][r] = 0.0f;
        }
    }
  }
  float best_v = best_vq[0];
  int best_i = best_iq[0];
  floatx16 acc = accq[0];
  if (KP > 1) {
    if (p > 0) {
      float* dst = red + ((p - 1) * EG + g) * 32 * PR;
#pragma unroll
      for (int r = 0; r < 16; ++r) dst[fm_mfma32_row(r, lane) * PR + col] = acc[r];
    }
    __syncthreads();
    if (p == 0 && g < nsub) {
      const int n0 = e_begin + 32 * g;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = fm_mfma32_row(r, lane);
        float v = acc[r];
#pragma unroll
        for (int pp = 1; pp < KP; ++pp) v = __fadd_rn(v, red[((pp - 1) * EG + g) * 32 * PR + row * PR + col]);
        const int entry = n0 + row;
        if (entry < e_end) {
          const float d = __fadd_rn(__fadd_rn(__fmul_rn(-2.0f, v), xq[0]), normS[entry - e_begin]);
          const float dist = dist_key(d);
          if (better(dist, entry, best_v, best_i)) best_v = dist, best_i = entry;
        }
      }
    }
  }
  best_vq[0] = best_v;
  best_iq[0] = best_i;
#pragma unroll
  for (int qt = 0; qt < QTN; ++qt) {
    const float ov = __shfl_xor(best_vq[qt], 32, 64);
    const int oi = __shfl_xor(best_iq[qt], 32, 64);
    if (better(ov, oi, best_vq[qt], best_iq[qt])) best_vq[qt] = ov, best_iq[qt] = oi;
    if (p == 0 && h == 0) bestv[g * RBT + col + 32 * qt] = best_vq[qt], besti[g * RBT + col + 32 * qt] = best_iq[qt];
  }
  __syncthreads();
  if (tid < RBT) {
    const long m = m0 + tid;
    float v = bestv[tid];
    int i = besti[tid];
#pragma unroll
    for (int gg = 1; gg < EG; ++gg)
      if (better(bestv[gg * RBT + tid], besti[gg * RBT + tid], v, i)) v = bestv[gg * RBT + tid], i = besti[gg * RBT + tid];
    if (m < a.M) {
      a.val[(long)chunk * a.M + m] = v;
      a.idx[(long)chunk * a.M + m] = i;
    }
  }
}

// ---------------------------------------------------------------------------
// Whole split encode in one persistent launch, for few rows (<= 4 tiles of 32
// rows: the B = 1 clips of up to ~10 s).  The step kernel above needs one
// launch per codebook and re-resolves the previous step's argmin in each of
// its blocks; here the residual chain of a (32-row tile, branch) pair stays
// in one group of CHAIN_BLOCKS blocks that steps through every codebook of
// the branch:
//   block b runs on XCD x = b % 8 (the dispatcher's round robin); tile t =
//   x / 2 owns XCDs 2t and 2t + 1, and of the 64 blocks j = b / 8 each XCD
//   holds for it, j < 32 serve the acoustic chain and j >= 32 the semantic
//   one (which ends after its first codebook, leaving each CU one acoustic
//   block with one wave per SIMD);  block q = 32 (x % 2) + j % 32 of a group
//   owns codebook entries [32 q, 32 q + 32), four waves = four 64-dim k-parts;
//   each step: distances of the 32 residual rows to the block's entries,
//   block argmin per row -> partial (value, index, step tag) stored
//   coherently -> every block polls the group's partials of its rows until
//   all carry the step's tag, resolves the argmin and subtracts the chosen
//   entry from its own copy of the residual (LDS), so residual rows never
//   leave the block and no separate barrier is needed.
// Partials are double-buffered by step parity: a block can only write step
// s + 2 after every block wrote step s + 1, i.e. after every block has read
// step s.  The tags of the zeroed slots (0) never match a step (>= 1).
// The arithmetic is rvq_step_mfma_kernel<256, 4>'s operation for operation
// (32x32x2 FP32 MFMA chains over four 64-dim k-parts summed in k-part order,
// |r|^2 over eight lanes per row, the same distance and residual rounding),
// so the codes are bit-identical to the per-step launches.  Block barriers
// order LDS only (lds_barrier), so the next codebook's fragment loads stay in
// flight across them.
constexpr int CHAIN_BLOCKS = 64;  // blocks per group: 64 x 32 entries
constexpr int CHAIN_GROUPS = 8;   // (tile, branch) pairs
constexpr int CHAIN_ENTRIES = CHAIN_BLOCKS * 32;
constexpr long CHAIN_SPIN = 1L << 20;  // polls before a wait gives up (~1 s)
constexpr size_t CHAIN_PARTIALS = (size_t)2 * CHAIN_GROUPS * CHAIN_BLOCKS * RB;
constexpr size_t CHAIN_WORKSPACE_BYTES = CHAIN_PARTIALS * 8 + 256;

struct ChainArgs {
  const float* x;   // [M][ld_x]: semantic input in columns [0, 256), acoustic in [256, 512)
  int ld_x, M, rows_per_batch, entries, batch_stride;
  int count[2];     // codebooks per branch
  const float* embeds[2];  // branch codebooks [count][entries][256]
  const float* norms[2];   // [count][entries]
  int64_t* codes[2];       // codebook 0 of the branch; codebook j at + j * rows_per_batch
  unsigned long long* partials;  // [2][CHAIN_GROUPS][CHAIN_BLOCKS][32], zeroed before the launch
  unsigned* status;        // counts blocks whose wait gave up (block 0 then recomputes alone)
  long spin_limit;         // polls before a wait gives up
};

__global__ __launch_bounds__(256, 4) void rvq_chain_kernel(ChainArgs a) {
  constexpr int DIM = 256, PX = DIM + 4, PR = RB + 1, CH = DIM / 32, PER = CHAIN_BLOCKS / 8;
  __shared__ __attribute__((aligned(16))) float Xs[RB * PX];  // residual rows
  __shared__ float xnS[RB];
  __shared__ float red[4][32 * PR];   // each wave's k-part dot products [p][entry][row]
  __shared__ float bestv[4][RB];      // per wave: best over its entries, per row
  __shared__ int besti[4][RB];
  __shared__ float normS[32];
  __shared__ int failS;

  const int x = blockIdx.x % 8, j = blockIdx.x / 8;
  const int tile = x >> 1, br = j >= 32 ? 0 : 1;
  const int g = tile * 2 + br, q = (x & 1) * 32 + (j & 31);
  const long m0 = (long)tile * RB;
  const int count = a.count[br];
  if (m0 >= a.M || count == 0) return;  // this pair has no work (the whole group returns)
  const float* __restrict__ embeds = a.embeds[br];
  const int tid = threadIdx.x, lane = tid & 63, p = tid >> 6;  // wave = k-part
  const int h = lane >> 5, col = lane & 31;
  const int e_begin = q * 32;
  const int kbase = p * 64;
  auto slot = [&](int s, int blk, int row) {
    return a.partials + (((long)(s & 1) * CHAIN_GROUPS + g) * CHAIN_BLOCKS + blk) * RB + row;
  };
  if (tid == 0) failS = 0;

  // Codebook fragment of this wave: entry eb + col, dims kbase + 32 h .. + 31
  // (rvq_step_mfma_kernel's load_piece); the slice's 32 norms ride along.
  floatx4 cur[8];
  float nrm = 0.0f;
  auto load_slice = [&](int jj, int eb) {
    const int entry = min(eb + col, a.entries - 1);
    const float* src = embeds + ((long)jj * a.entries + entry) * DIM + kbase + 32 * h;
#pragma unroll
    for (int u = 0; u < 8; ++u) cur[u] = *reinterpret_cast<const floatx4*>(src + 4 * u);
    if (tid < 32) nrm = eb + tid < a.entries ? a.norms[br][(long)jj * a.entries + eb + tid] : 0.0f;
  };
  auto load_piece = [&](int jj) { load_slice(jj, e_begin); };
  // Distances of the 32 residual rows (Xs) to the 32 entries in `cur`, this
  // wave's k-part: entries on the MFMA rows.
  auto distances = [&]() {
    floatx16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int jj = 0; jj < 8; ++jj) {
      const floatx4 b4 = *reinterpret_cast<const floatx4*>(Xs + col * PX + kbase + 32 * h + 4 * jj);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc = fm_mfma32(cur[jj][e], b4[e], acc);
    }
    // 19 wait states before anything reads the accumulators (a 16-pass
    // 32x32 MFMA needs 18).  The compiler's own count missed two reads
    // placed behind a branch, so the wait is explicit, and the tile passes
    // through the asm so that no read can move above it.
    asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 2" : "+a"(acc));
    return acc;
  };
  // Every wave publishes its k-part; then wave p finishes entries
  // 8 (r / 4) + 4 h + (r % 4) for r = 4 p .. 4 p + 3 (four of the sixteen
  // accumulator rows), summing the k-parts in order 0..3, and leaves its best
  // entry of slice `eb` per row in bestv / besti[p] (norms from normS).
  auto slice_best = [&](const floatx16& acc, int eb) {
#pragma unroll
    for (int r = 0; r < 16; ++r) red[p][fm_mfma32_row(r, lane) * PR + col] = acc[r];
    lds_barrier();
    float best_v = INFINITY;
    int best_i = 0x7fffffff;
    const float xq = xnS[col];
#pragma unroll
    for (int rr = 0; rr < 4; ++rr) {
      const int row = fm_mfma32_row(4 * p + rr, lane);
      float v = red[0][row * PR + col];
#pragma unroll
      for (int pp = 1; pp < 4; ++pp) v = __fadd_rn(v, red[pp][row * PR + col]);
      const int entry = eb + row;
      if (entry < a.entries) {
        const float d = __fadd_rn(__fadd_rn(__fmul_rn(-2.0f, v), xq), normS[row]);
        const float dist = dist_key(d);
        if (better(dist, entry, best_v, best_i)) best_v = dist, best_i = entry;
      }
    }
    const float ov = __shfl_xor(best_v, 32, 64);
    const int oi = __shfl_xor(best_i, 32, 64);
    if (better(ov, oi, best_v, best_i)) best_v = ov, best_i = oi;
    if (h == 0) bestv[p][col] = best_v, besti[p][col] = best_i;
    lds_barrier();
  };
  // Row `row`'s best over the four waves of the last slice_best.
  auto block_best = [&](int row, float& v, int& i) {
    v = bestv[0][row];
    i = besti[0][row];
#pragma unroll
    for (int w = 1; w < 4; ++w)
      if (better(bestv[w][row], besti[w][row], v, i)) v = bestv[w][row], i = besti[w][row];
  };
  load_piece(0);

  // Residual rows of step 0: the branch's input columns (eight lanes per row).
  {
    const int r = tid >> 3, pt = tid & 7;
    const long m = m0 + r;
    const bool valid = m < a.M;
    const float* xr = a.x + min(m, (long)a.M - 1) * a.ld_x + br * DIM;
    float xn = 0.0f;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      floatx4 xv = *reinterpret_cast<const floatx4*>(xr + 4 * (pt + 8 * u));
      if (!valid) xv = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int e = 0; e < 4; ++e) xn = fmaf(xv[e], xv[e], xn);
      *reinterpret_cast<floatx4*>(Xs + r * PX + 4 * (pt + 8 * u)) = xv;
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) xn += __shfl_xor(xn, o, 64);
    if (pt == 0) xnS[r] = xn;
  }

  int s_fail = -1;  // step at which a wait of this block gave up
  for (int s = 0; s <= count; ++s) {
    if (s > 0) {
      // Only block 0 of the group needs the last step's codes.
      if (s == count && q != 0) break;
      // Resolve step s - 1: eight lanes per row, each polling PER partials
      // until all carry tag s, then a shuffle reduction (`better` is a
      // total order, so the grouping does not change the result).
      const int r = tid >> 3, pt = tid & 7;
      // Each lane first polls one of its partials, then loads all of them
      // (a full re-poll only if one is still missing): eight times fewer
      // coherent loads while waiting than polling all (measured 49.7 vs
      // 56.1 us per call at C2; pipelined polls: 60 us).
      unsigned long long pv[PER] = {};  // (a wait that gives up resolves zeros: index 0)
      bool ready = false;
      for (long spin = 0; !ready && spin < a.spin_limit; ++spin) {
        if ((unsigned)(fm_load64_coherent(slot(s - 1, pt + 8 * (PER - 1), r)) >> 48) != (unsigned)s) continue;
#pragma unroll
        for (int u = 0; u < PER; ++u) pv[u] = fm_load64_coherent(slot(s - 1, pt + 8 * u, r));
        ready = true;
#pragma unroll
        for (int u = 0; u < PER; ++u) ready &= (unsigned)(pv[u] >> 48) == (unsigned)s;
      }
      if (!ready) failS = 1;
      float bv = INFINITY;
      int bi = 0x7fffffff;
#pragma unroll
      for (int u = 0; u < PER; ++u) {
        const float v = __uint_as_float((unsigned)pv[u]);
        const int i = (int)((pv[u] >> 32) & 0xffff);
        if (better(v, i, bv, bi)) bv = v, bi = i;
      }
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) {
        const float ov = __shfl_xor(bv, o, 64);
        const int oi = __shfl_xor(bi, o, 64);
        if (better(ov, oi, bv, bi)) bv = ov, bi = oi;
      }
      bi = code_index(bi, a.entries);
      const long m = m0 + r;
      if (q == 0 && pt == 0 && m < a.M) {
        const long b = m / a.rows_per_batch, t = m - b * a.rows_per_batch;
        a.codes[br][(long)(s - 1) * a.rows_per_batch + b * a.batch_stride + t] = bi;
      }
      if (s == count) {
        // The last resolve (block 0 only): one barrier per call to learn
        // whether one of its waits gave up.
        lds_barrier();
        if (failS) s_fail = s;
        break;
      }
      // residual_s = residual_{s-1} - e_{s-1}[code], and its |.|^2.
      const float* er = embeds + ((long)(s - 1) * a.entries + bi) * DIM;
      floatx4 ev[CH];
#pragma unroll
      for (int u = 0; u < CH; ++u) ev[u] = *reinterpret_cast<const floatx4*>(er + 4 * (pt + 8 * u));
      const bool valid = m < a.M;
      float xn = 0.0f;
#pragma unroll
      for (int u = 0; u < CH; ++u) {
        floatx4 xv = *reinterpret_cast<const floatx4*>(Xs + r * PX + 4 * (pt + 8 * u));
#pragma unroll
        for (int e = 0; e < 4; ++e) xv[e] = __fsub_rn(xv[e], ev[u][e]);
        if (!valid) xv = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
        for (int e = 0; e < 4; ++e) xn = fmaf(xv[e], xv[e], xn);
        *reinterpret_cast<floatx4*>(Xs + r * PX + 4 * (pt + 8 * u)) = xv;
      }
#pragma unroll
      for (int o = 1; o < 8; o <<= 1) xn += __shfl_xor(xn, o, 64);
      if (pt == 0) xnS[r] = xn;
    }
    if (tid < 32) normS[tid] = nrm;
    lds_barrier();
    if (failS) {
      s_fail = s;
      break;
    }

    // Distances: 32 entries (A, from registers) x 32 rows (B, from LDS), this wave's k-part.
    const floatx16 acc = distances();
    // Next codebook's fragment and norms go out now; their latency hides
    // behind the reduction and the resolve (the last step reloads its own
    // piece: no branch between the MFMAs and the accumulator reads).
    load_piece(min(s + 1, count - 1));
    slice_best(acc, e_begin);
    if (tid < RB) {
      float v;
      int i;
      block_best(tid, v, i);
      // A block with no entries in range publishes +inf (index 0xffff).
      if (i > 0xffff) i = 0xffff;
      fm_store64_coherent(slot(s, q, tid), ((unsigned long long)(s + 1) << 48) |
                                               ((unsigned long long)(unsigned)i << 32) | __float_as_uint(v));
    }
  }
  if (s_fail < 0) return;
  if (tid == 0) __hip_atomic_fetch_add(a.status, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  // A wait gave up (a block of the group never became resident in time,
  // say).  Only block 0 writes codes: the others leave, and block 0 (whose
  // own waits then give up too, if they had not) computes the whole chain
  // again alone, from the input rows, with every slice's distances and the
  // arithmetic above, so the codes are the ones the group would have
  // resolved.  Slower, never wrong; every wait is bounded, so the grid
  // drains.
  if (q != 0) return;
  const int r = tid >> 3, pt = tid & 7;
  const long m = m0 + r;
  const bool valid = m < a.M;
  {
    const float* xr = a.x + min(m, (long)a.M - 1) * a.ld_x + br * DIM;
    float xn = 0.0f;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      floatx4 xv = *reinterpret_cast<const floatx4*>(xr + 4 * (pt + 8 * u));
      if (!valid) xv = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int e = 0; e < 4; ++e) xn = fmaf(xv[e], xv[e], xn);
      *reinterpret_cast<floatx4*>(Xs + r * PX + 4 * (pt + 8 * u)) = xv;
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) xn += __shfl_xor(xn, o, 64);
    if (pt == 0) xnS[r] = xn;
  }
  for (int jj = 0; jj < count; ++jj) {
    float fv = INFINITY;
    int fi = 0x7fffffff;
    for (int qs = 0; qs * 32 < a.entries; ++qs) {
      load_slice(jj, qs * 32);
      if (tid < 32) normS[tid] = nrm;
      lds_barrier();
      slice_best(distances(), qs * 32);
      if (tid < RB) {
        float v;
        int i;
        block_best(tid, v, i);
        if (better(v, i, fv, fi)) fv = v, fi = i;
      }
    }
    if (tid < RB) besti[0][tid] = fi;
    lds_barrier();
    const int bi = code_index(besti[0][r], a.entries);
    if (pt == 0 && valid) {
      const long b = m / a.rows_per_batch, t = m - b * a.rows_per_batch;
      a.codes[br][(long)jj * a.rows_per_batch + b * a.batch_stride + t] = bi;
    }
    if (jj + 1 == count) break;
    const float* er = embeds + ((long)jj * a.entries + bi) * DIM;
    float xn = 0.0f;
#pragma unroll
    for (int u = 0; u < CH; ++u) {
      const floatx4 ev = *reinterpret_cast<const floatx4*>(er + 4 * (pt + 8 * u));
      floatx4 xv = *reinterpret_cast<const floatx4*>(Xs + r * PX + 4 * (pt + 8 * u));
#pragma unroll
      for (int e = 0; e < 4; ++e) xv[e] = __fsub_rn(xv[e], ev[e]);
      if (!valid) xv = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int e = 0; e < 4; ++e) xn = fmaf(xv[e], xv[e], xn);
      *reinterpret_cast<floatx4*>(Xs + r * PX + 4 * (pt + 8 * u)) = xv;
    }
#pragma unroll
    for (int o = 1; o < 8; o <<= 1) xn += __shfl_xor(xn, o, 64);
    if (pt == 0) xnS[r] = xn;
    lds_barrier();
  }
}

// Zeroes the chain kernel's partial slots (so no stale tag can match) and its
// status word: a kernel, not a memset node, so the pair can be captured in a
// hipGraph.
__global__ __launch_bounds__(256) void rvq_chain_reset_kernel(unsigned long long* partials, long n) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;
  if (i < n) partials[i] = 0ull;
}

// Resolves the last step: 8 lanes per row (32 rows per block).
__global__ __launch_bounds__(256) void rvq_finalize_kernel(const float* val, const int* idx,
                                                           int chunks, int M, int64_t* codes,
                                                           int rows_per_batch, int batch_stride,
                                                           int entries) {
  const long m = (long)blockIdx.x * 32 + (threadIdx.x >> 3);
  const int pt = threadIdx.x & 7;
  float bv;
  int bi;
  resolve8(val, idx, chunks, M, min(m, (long)M - 1), pt, bv, bi);
  if (m >= M || pt != 0) return;
  const long b = m / rows_per_batch, t = m - b * rows_per_batch;
  codes[b * batch_stride + t] = code_index(bi, entries);
}

// embed = embed_sum / max(usage, eps); transposed copy; squared norms.
__global__ __launch_bounds__(256) void rvq_prepare_kernel(const float* embed_sum, const float* usage,
                                                          int entries, int dim, float eps,
                                                          float* embed, float* embed_t,
                                                          float* norms) {
  const int e = blockIdx.x;
  const float u = fmaxf(usage[e], eps);
  float s = 0.0f;
  for (int k = threadIdx.x; k < dim; k += 256) {
    const float v = embed_sum[(long)e * dim + k] / u;
    embed[(long)e * dim + k] = v;
    embed_t[(long)k * entries + e] = v;
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    for (int k = 0; k < dim; ++k) {
      const float v = embed[(long)e * dim + k];
      s = fmaf(v, v, s);
    }
    norms[e] = s;
  }
}

// out[m][0:dim] = 0 + E_0[c_0];  out[m][dim:2dim] = ((0 + E_1[c_1]) + E_2[c_2]) + ...
// Codebook j lives at embeds + j * entries * dim.  Out-of-range codes yield NaN.
__global__ __launch_bounds__(256) void rvq_decode_kernel(const int64_t* codes, int nq, int n_sem,
                                                         int rows_per_batch, long M,
                                                         const float* embeds, int entries, int dim,
                                                         float* out) {
  const long e = (long)blockIdx.x * 256 + threadIdx.x;
  if (e >= M * dim) return;
  const long m = e / dim;
  const int k = (int)(e - m * dim);
  const long b = m / rows_per_batch, t = m - b * rows_per_batch;
  const int64_t* cp = codes + b * (long)nq * rows_per_batch + t;
  float sem = 0.0f, ac = 0.0f;
  for (int j = 0; j < nq; ++j) {
    const int64_t c = cp[(long)j * rows_per_batch];
    float v = (c >= 0 && c < entries) ? embeds[((long)j * entries + c) * dim + k] : NAN;
    if (j < n_sem) sem = __fadd_rn(sem, v);
    else ac = __fadd_rn(ac, v);
  }
  out[m * 2 * dim + k] = sem;
  out[m * 2 * dim + dim + k] = ac;
}

size_t step_lds_bytes(int dim) {
  return (size_t)dim * (RB + 1) * 4 + (size_t)KSL * PB * 4 + RB * 4 + 4 * RB * 4 + 4 * RB * 4 +
         RB * 4;
}

// Launch plan shared by every step of an encode: fast MFMA kernel with KP
// k-parts per 32-entry sub-tile while the launch stays within ~1024 blocks,
// else 128-entry (or larger) chunks.  General kernel: chunks doubling until
// the launch has 512 blocks, multiples of NT entries.
struct RvqPlan {
  bool fast;
  int kp, qt, chunks, ce, row_blocks;
  size_t lds;
};

RvqPlan rvq_plan(int rows, int dim, int entries) {
  RvqPlan pl{};
  pl.row_blocks = (rows + RB - 1) / RB;
  pl.fast = (dim == 64 || dim == 128 || dim == 256);
  pl.chunks = 1;
  pl.kp = 1;
  pl.qt = 1;
  constexpr int blocks_cap = 1024;
  if (pl.fast) {
    const int sub = (entries + 31) / 32;
    if (dim >= 256 && sub <= kMaxChunks && pl.row_blocks * sub <= blocks_cap) {
      pl.kp = 4, pl.chunks = sub;
    } else if (dim >= 128 && (sub + 1) / 2 <= kMaxChunks && pl.row_blocks * ((sub + 1) / 2) <= blocks_cap) {
      pl.kp = 2, pl.chunks = (sub + 1) / 2;
    } else {
      // Many rows: 64-row blocks (two query tiles per codebook fragment).
      if (rows >= 1024 && entries <= kQt2MaxChunkEntries) {
        pl.qt = 2;
        pl.row_blocks = (rows + 2 * RB - 1) / (2 * RB);
      }
      int per = 128;
      while ((entries + per - 1) / per > kMaxChunks || pl.row_blocks * ((entries + per - 1) / per) > blocks_cap) {
        if (per >= entries) break;
        per *= 2;
      }
      pl.chunks = (entries + per - 1) / per;
    }
  } else {
    while (pl.chunks < 16 && pl.row_blocks * pl.chunks < 512 && entries / (pl.chunks * 2) >= NT) pl.chunks *= 2;
  }
  const int chunk_entries = pl.fast ? (pl.kp == 4 ? 32 : pl.kp == 2 ? 64 : (entries + pl.chunks - 1) / pl.chunks)
                                    : ((entries + pl.chunks - 1) / pl.chunks + NT - 1) / NT * NT;
  pl.ce = pl.fast && pl.kp == 1 ? (chunk_entries + 31) / 32 * 32 : chunk_entries;
  // Dynamic LDS (64-row blocks use a static array instead).
  pl.lds = pl.fast ? (pl.qt == 2 ? 0 : ((size_t)RB * (dim + 4) + RB + 2 * 4 * RB + 3 * 32 * (RB + 1) + pl.ce) * 4)
                   : step_lds_bytes(dim);
  return pl;
}

// One branch's buffers: two residual / partial sets used alternately by the steps.
struct RvqBranch {
  const float* x;
  int ld_x, count;
  const float *embeds, *embeds_t, *norms;
  int64_t* codes;
  float* resid[2];
  float* val[2];
  int* idx[2];
};

RvqBranch rvq_branch(const float* x, int ld_x, int count, const float* embeds, const float* embeds_t,
                     const float* norms, int64_t* codes, void* workspace, int rows, int dim) {
  RvqBranch br{x, ld_x, count, embeds, embeds_t, norms, codes, {}, {}, {}};
  char* ws = static_cast<char*>(workspace);
  br.resid[0] = reinterpret_cast<float*>(ws);
  br.resid[1] = br.resid[0] + (size_t)rows * dim;
  ws += (size_t)2 * rows * dim * sizeof(float);
  br.val[0] = reinterpret_cast<float*>(ws);
  br.val[1] = br.val[0] + (size_t)kMaxChunks * rows;
  ws += (size_t)2 * kMaxChunks * rows * sizeof(float);
  br.idx[0] = reinterpret_cast<int*>(ws);
  br.idx[1] = br.idx[0] + (size_t)kMaxChunks * rows;
  return br;
}

// Step j of a branch (j == count: resolve the last codebook only).
StepArgs rvq_step_args(const RvqBranch& br, int j, const RvqPlan& pl, int rows, int rows_per_batch,
                       int dim, int entries, int batch_stride) {
  StepArgs a{};
  const int cur = j & 1, prev = cur ^ 1;
  if (j == 0) {
    a.resid_in = br.x;
    a.ld_in = br.ld_x;
  } else {
    a.resid_in = (j == 1) ? br.x : br.resid[prev];
    a.ld_in = (j == 1) ? br.ld_x : dim;
    a.prev_embed = br.embeds + (size_t)(j - 1) * entries * dim;
    a.prev_val = br.val[prev];
    a.prev_idx = br.idx[prev];
    a.resid_out = j < br.count ? br.resid[cur] : nullptr;
    a.prev_codes = br.codes + (size_t)(j - 1) * rows_per_batch;
  }
  if (j < br.count) {
    a.embed_t = br.embeds_t + (size_t)j * entries * dim;
    a.norms = br.norms + (size_t)j * entries;
    a.val = br.val[cur];
    a.idx = br.idx[cur];
  }
  a.M = rows; a.dim = dim; a.entries = entries; a.chunk_entries = pl.ce;
  a.chunks = pl.chunks; a.rows_per_batch = rows_per_batch; a.batch_stride = batch_stride;
  return a;
}

int launch_fast_step(const RvqPlan& pl, int dim, dim3 grid, const StepArgs& a0, const float* e0,
                     const StepArgs& a1, const float* e1, hipStream_t stream) {
#define FM_RVQ(D, K) \
  hipLaunchKernelGGL((rvq_step_mfma_kernel<D, K>), grid, dim3(256), pl.lds, stream, a0, e0, a1, e1)
#define FM_RVQ2(D) \
  hipLaunchKernelGGL((rvq_step_mfma_kernel<D, 1, 2>), grid, dim3(256), 0, stream, a0, e0, a1, e1)
  if (pl.qt == 2) {
    if (dim == 256) FM_RVQ2(256);
    else if (dim == 128) FM_RVQ2(128);
    else FM_RVQ2(64);
#undef FM_RVQ2
  } else if (dim == 256 && pl.kp == 4) FM_RVQ(256, 4);
  else if (dim == 256 && pl.kp == 2) FM_RVQ(256, 2);
  else if (dim == 256) FM_RVQ(256, 1);
  else if (dim == 128 && pl.kp == 2) FM_RVQ(128, 2);
  else if (dim == 128) FM_RVQ(128, 1);
  else FM_RVQ(64, 1);
#undef FM_RVQ
  return (int)hipGetLastError();
}

// The persistent chain needs all CHAIN_GROUPS * CHAIN_BLOCKS blocks resident
// at once (each waits on every block of its group): two per CU, so at least
// half as many CUs as blocks.  FM_RVQ_CHAIN=0 in the
// environment selects the per-step launches instead (for comparisons).
bool chain_eligible(int rows, int dim, int entries) {
  if (dim != 256 || entries > CHAIN_ENTRIES || rows > (CHAIN_GROUPS / 2) * RB) return false;
  static const bool enabled = [] {
    const char* v = getenv("FM_RVQ_CHAIN");
    return !(v && v[0] == '0');
  }();
  if (!enabled) return false;
  constexpr int kMaxDev = 64;
  static int cus[kMaxDev] = {};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDev) return false;
  if (cus[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return false;
    cus[dev] = n;
  }
  return 2 * cus[dev] >= CHAIN_GROUPS * CHAIN_BLOCKS;
}

bool rvq_args_ok(const float* x, int ld_x, int rows, int rows_per_batch, int dim, int entries,
                 const float* embeds, const float* embeds_t, const float* norms, const int64_t* codes) {
  return x && embeds && embeds_t && norms && codes && rows >= 0 && dim > 0 && dim % 4 == 0 &&
         ld_x % 4 == 0 && entries > 0 && rows_per_batch > 0 && ld_x >= dim;
}

}  // namespace

extern "C" {

int fm_rvq_prepare_codebook(const float* embed_sum, const float* cluster_usage, int entries,
                            int dim, float eps, float* embed, float* embed_t, float* norms,
                            hipStream_t stream) {
  if (!embed_sum || !cluster_usage || !embed || !embed_t || !norms || entries <= 0 || dim <= 0)
    return FM_BAD_ARGUMENT;
  hipLaunchKernelGGL(rvq_prepare_kernel, dim3(entries), dim3(256), 0, stream, embed_sum,
                     cluster_usage, entries, dim, eps, embed, embed_t, norms);
  return (int)hipGetLastError();
}

// Partials workspace needed by fm_rvq_encode, in bytes.
size_t fm_rvq_workspace_bytes(int rows, int dim, int entries) {
  (void)entries;
  const int chunks = kMaxChunks;
  return (size_t)2 * rows * dim * sizeof(float) + (size_t)2 * chunks * rows * (sizeof(float) + sizeof(int)) + 256;
}

// Encodes one RVQ branch: ``count`` codebooks applied to rows x[m] (pitch ld_x).
// embeds / embeds_t / norms hold the branch's codebooks contiguously
// ([count][entries][dim], [count][dim][entries], [count][entries]).
// codes: int64 base of codebook 0's codes; row (b, t) of codebook j lands at
// codes[b * batch_stride + j * rows_per_batch + t].
int fm_rvq_encode(const float* x, int ld_x, int rows, int rows_per_batch, int dim, int entries,
                  int count, const float* embeds, const float* embeds_t, const float* norms,
                  int64_t* codes, int batch_stride, void* workspace, size_t workspace_bytes,
                  hipStream_t stream) {
  if (!rvq_args_ok(x, ld_x, rows, rows_per_batch, dim, entries, embeds, embeds_t, norms, codes) ||
      count <= 0)
    return FM_BAD_ARGUMENT;
  if (rows == 0) return FM_OK;
  if (!workspace || workspace_bytes < fm_rvq_workspace_bytes(rows, dim, entries))
    return FM_WORKSPACE_TOO_SMALL;
  const RvqPlan pl = rvq_plan(rows, dim, entries);
  if (pl.lds > 64 * 1024) return FM_UNSUPPORTED;
  const RvqBranch br = rvq_branch(x, ld_x, count, embeds, embeds_t, norms, codes, workspace, rows, dim);
  const dim3 grid(pl.row_blocks, pl.chunks);
  for (int j = 0; j < count; ++j) {
    const StepArgs a = rvq_step_args(br, j, pl, rows, rows_per_batch, dim, entries, batch_stride);
    int e;
    if (!pl.fast) {
      hipLaunchKernelGGL(rvq_step_kernel, grid, dim3(256), pl.lds, stream, a);
      e = (int)hipGetLastError();
    } else {
      e = launch_fast_step(pl, dim, grid, a, br.embeds + (size_t)j * entries * dim, a, nullptr, stream);
    }
    if (e != hipSuccess) return e;
  }
  const int last = (count - 1) & 1;
  hipLaunchKernelGGL(rvq_finalize_kernel, dim3((rows + 31) / 32), dim3(256), 0, stream,
                     br.val[last], br.idx[last], pl.chunks, rows,
                     codes + (size_t)(count - 1) * rows_per_batch, rows_per_batch, batch_stride, entries);
  return (int)hipGetLastError();
}

size_t fm_rvq_split_workspace_bytes(int rows, int dim, int entries) {
  return std::max(2 * fm_rvq_workspace_bytes(rows, dim, entries), CHAIN_WORKSPACE_BYTES);
}

// Both branches of the split quantizer in shared launches: launch s runs
// step s of every branch that still has one (blockIdx.z = branch) and
// resolves the last codebook of a branch whose chain ended at s - 1.
// x: semantic input in columns [0, dim), acoustic input in [dim, 2*dim).
// Codebooks 0 .. n_semantic-1 are the semantic branch, the next n_acoustic
// the acoustic one, all contiguous in embeds / embeds_t / norms.
int fm_rvq_encode_split(const float* x, int ld_x, int rows, int rows_per_batch, int dim, int entries,
                        int n_semantic, int n_acoustic, const float* embeds, const float* embeds_t,
                        const float* norms, int64_t* codes, int batch_stride, void* workspace,
                        size_t workspace_bytes, hipStream_t stream) {
  if (!rvq_args_ok(x, ld_x, rows, rows_per_batch, dim, entries, embeds, embeds_t, norms, codes) ||
      n_semantic < 0 || n_acoustic < 0 || n_semantic + n_acoustic <= 0 || ld_x < 2 * dim)
    return FM_BAD_ARGUMENT;
  if (rows == 0) return FM_OK;
  const size_t one = fm_rvq_workspace_bytes(rows, dim, entries);
  if (!workspace || workspace_bytes < 2 * one) return FM_WORKSPACE_TOO_SMALL;
  const size_t cb = (size_t)entries * dim;
  char* ws = static_cast<char*>(workspace);
  const bool fast = (dim == 64 || dim == 128 || dim == 256);
  if (!fast || n_semantic == 0 || n_acoustic == 0) {
    // One chain (or the general kernel): the branches run one after the other.
    if (n_semantic > 0) {
      const int e = fm_rvq_encode(x, ld_x, rows, rows_per_batch, dim, entries, n_semantic, embeds,
                                  embeds_t, norms, codes, batch_stride, ws, one, stream);
      if (e != FM_OK) return e;
    }
    if (n_acoustic > 0)
      return fm_rvq_encode(x + dim, ld_x, rows, rows_per_batch, dim, entries, n_acoustic,
                           embeds + n_semantic * cb, embeds_t + n_semantic * cb,
                           norms + (size_t)n_semantic * entries,
                           codes + (size_t)n_semantic * rows_per_batch, batch_stride, ws + one, one,
                           stream);
    return FM_OK;
  }
  // (A workspace sized for the per-step launches only takes them.)
  if (workspace_bytes >= CHAIN_WORKSPACE_BYTES && chain_eligible(rows, dim, entries)) {
    // Few rows: the whole chain of both branches in one persistent launch.
    ChainArgs c{};
    c.x = x; c.ld_x = ld_x; c.M = rows; c.rows_per_batch = rows_per_batch; c.entries = entries;
    c.batch_stride = batch_stride;
    c.count[0] = n_semantic; c.count[1] = n_acoustic;
    c.embeds[0] = embeds; c.embeds[1] = embeds + n_semantic * cb;
    c.norms[0] = norms; c.norms[1] = norms + (size_t)n_semantic * entries;
    c.codes[0] = codes; c.codes[1] = codes + (size_t)n_semantic * rows_per_batch;
    c.partials = reinterpret_cast<unsigned long long*>(ws);
    c.status = reinterpret_cast<unsigned*>(ws + CHAIN_PARTIALS * 8);
    // FM_RVQ_CHAIN_SPIN (tests) lowers the polls a wait may take before its
    // block goes solo; 0 sends every block down that path.
    c.spin_limit = CHAIN_SPIN;
    if (const char* v = getenv("FM_RVQ_CHAIN_SPIN")) c.spin_limit = std::max(0L, atol(v));
    const long words = (long)CHAIN_PARTIALS + 1;  // the status word follows the slots
    hipLaunchKernelGGL(rvq_chain_reset_kernel, dim3((unsigned)((words + 255) / 256)), dim3(256), 0, stream,
                       c.partials, words);
    hipLaunchKernelGGL(rvq_chain_kernel, dim3(CHAIN_GROUPS * CHAIN_BLOCKS), dim3(256), 0, stream, c);
    return (int)hipGetLastError();
  }
  const RvqPlan pl = rvq_plan(rows, dim, entries);
  if (pl.lds > 64 * 1024) return FM_UNSUPPORTED;
  RvqBranch br[2] = {
      rvq_branch(x, ld_x, n_semantic, embeds, embeds_t, norms, codes, ws, rows, dim),
      rvq_branch(x + dim, ld_x, n_acoustic, embeds + n_semantic * cb, embeds_t + n_semantic * cb,
                 norms + (size_t)n_semantic * entries, codes + (size_t)n_semantic * rows_per_batch,
                 ws + one, rows, dim)};
  const int steps = std::max(n_semantic, n_acoustic);
  for (int s = 0; s <= steps; ++s) {
    // Branches active at launch s: step s (s < count) or the resolve of the last one (s == count).
    int act[2], na = 0;
    bool any_step = false;
    for (int b = 0; b < 2; ++b)
      if (s <= br[b].count) {
        act[na++] = b;
        any_step |= s < br[b].count;
      }
    if (na == 0) continue;
    const StepArgs a0 = rvq_step_args(br[act[0]], s, pl, rows, rows_per_batch, dim, entries, batch_stride);
    const StepArgs a1 = na > 1 ? rvq_step_args(br[act[1]], s, pl, rows, rows_per_batch, dim, entries, batch_stride) : a0;
    const float* e0 = s < br[act[0]].count ? br[act[0]].embeds + (size_t)s * cb : nullptr;
    const float* e1 = na > 1 && s < br[act[1]].count ? br[act[1]].embeds + (size_t)s * cb : nullptr;
    const dim3 grid(pl.row_blocks, any_step ? pl.chunks : 1, na);
    const int e = launch_fast_step(pl, dim, grid, a0, e0, a1, e1, stream);
    if (e != hipSuccess) return e;
  }
  return FM_OK;
}

int fm_rvq_decode(const int64_t* codes, int batch, int num_codebooks, int frames,
                  int num_semantic, const float* embeds, int entries, int dim, float* out,
                  hipStream_t stream) {
  if (!codes || !embeds || !out || batch < 0 || frames < 0 || num_codebooks <= 0 ||
      num_semantic < 0 || entries <= 0 || dim <= 0)
    return FM_BAD_ARGUMENT;
  const long M = (long)batch * frames;
  if (M == 0) return FM_OK;
  const long total = M * dim;
  hipLaunchKernelGGL(rvq_decode_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0,
                     stream, codes, num_codebooks, num_semantic, frames, M, embeds, entries, dim,
                     out);
  return (int)hipGetLastError();
}

}  // extern "C"

// ---------------------------------------------------------------------------
// Allocation-free split encode.  The step partials and residual ping-pong
// buffers live in a fixed device array instead of a caller workspace, so the
// entry point makes no allocation of any kind (for hipGraph capture, serving
// loops and harnesses that forbid hipMalloc).  Each GPU the library runs on
// holds its own copy of the array until the process ends.  Every call on a
// GPU shares that GPU's array: calls that overlap on one GPU (two streams, two
// threads) race and must be serialised by the caller.  Nothing in the array
// needs clearing between calls: every step writes all the partials and
// residual rows the next step reads before it reads them.

namespace {
constexpr size_t kNoAllocScratchBytes = size_t(48) << 20;  // 8,190 rows of 256-dim codebooks
constexpr int kMaxDevices = 64;
}  // namespace

static __device__ __align__(256) unsigned char scratch[kNoAllocScratchBytes];

namespace {

std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The device address of ``scratch`` on the current device (looked up once per
// device; the host-side name is only a stand-in for it).
int scratch_on_current_device(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return FM_UNSUPPORTED;
  std::lock_guard<std::mutex> guard(g_scratch_mutex);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (!ptr) return FM_UNSUPPORTED;
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return FM_OK;
}

}  // namespace

extern "C" {

size_t fm_rvq_noalloc_scratch_bytes(void) { return kNoAllocScratchBytes; }

int fm_rvq_encode_split_noalloc(const float* x, int ld_x, int rows, int rows_per_batch, int dim,
                                int entries, int n_semantic, int n_acoustic, const float* embeds,
                                const float* embeds_t, const float* norms, int64_t* codes,
                                int batch_stride, hipStream_t stream) {
  if (!rvq_args_ok(x, ld_x, rows, rows_per_batch, dim, entries, embeds, embeds_t, norms, codes) ||
      n_semantic < 0 || n_acoustic < 0 || n_semantic + n_acoustic <= 0 || ld_x < 2 * dim)
    return FM_BAD_ARGUMENT;
  if (rows == 0) return FM_OK;
  if (fm_rvq_split_workspace_bytes(rows, dim, entries) > kNoAllocScratchBytes)
    return FM_SCRATCH_LIMIT;
  void* ptr = nullptr;
  const int e = scratch_on_current_device(&ptr);
  if (e != FM_OK) return e;
  return fm_rvq_encode_split(x, ld_x, rows, rows_per_batch, dim, entries, n_semantic, n_acoustic,
                             embeds, embeds_t, norms, codes, batch_stride, ptr,
                             kNoAllocScratchBytes, stream);
}

}  // extern "C"
