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
// (replicate padding).  B is the packed weight W^T [N, K] (k contiguous).
//
// Fast kernel (C_in and K multiples of 4): both operands are staged in LDS
// k-contiguous (row pitch BK + 4 floats) with 16-byte writes, double-buffered.
// The MFMA k-slot of lane half h at step 4q+e carries k = (BK/2)h + 4q + e,
// so every lane fetches its A and B fragments for four MFMAs with one 16-byte
// LDS read each.  Tiles (256 threads; k-tile BK = 64 for the large tiles so a
// k-tile's MFMA work outlasts the next tile's global-load latency):
//   256x128 / 256x64 (8 waves of 64x64 / 64x32, one k-tile prefetched in
//   registers), 128x128 (2x2 waves of 64x64), 128x64 (4x1 of 32x64),
//   128x32 (4x1 of 32x32);
//   32x64 with the four waves splitting K (summed through LDS in wave order)
//   when the large tiles cannot fill the GPU, plus global K-splits summed in
//   split order by a second kernel for very long K.
// Long-K contractions with few rows (the 12.5-25 Hz end of the SEANet stacks)
// take 64x64 / 32x32 tiles of 16x16x4 MFMA chains with BK = 128 (gemm_mid),
// or 256x64 tiles, split along K to a few hundred blocks.  All sums are in a
// fixed order, so results are deterministic.
// Blocks are renumbered so consecutive tiles of one row band land on one XCD
// (dispatch assigns block i to XCD i % 8), keeping the band's A rows in that
// XCD's L2.
// A scalar generic kernel covers the remaining shapes (C_in or K not a
// multiple of 4: the 1-channel first convolution and tiny test configs).

#include <cstdio>
#include <type_traits>

#include "fm_common.h"

extern "C" int fm_apply_rope(float* x, long rows, int ld, int rope_cols, int head_dim,
                             const float* cos_table, const float* sin_table, int rows_per_seq,
                             hipStream_t stream);

namespace {

struct GemmArgs {
  const float* x;
  const float* w;  // W^T [N][K]
  const float* bias;
  const float* res;
  const float* scale;
  float* y;
  float* partial;  // global split-K partials [splits][M][N], or null
  int batch, L_in, C_in, rows, rs, padL, K, N, y_rows, bias_len, k_split, flags;
  FmDivisor rows_div;  // division by `rows` (set by run_gemm)
  // FM_EPI_ROPE: cos/sin tables [*][64] at position row % rows_per_seq for
  // output columns < rope_cols (heads of 64 columns).
  const float* rope_cos;
  const float* rope_sin;
  int rope_cols, rows_per_seq;
  FmDivisor seq_div;  // division by `rows_per_seq` (set by run_gemm)
};

constexpr int KT = 32;  // k granularity of K-splits (every tile's BK divides it or is 64)
constexpr int NTHREADS = 256;

FM_DEVICE float epilogue_v(float v, float bias, float res, float scale, int flags) {
  v = __fadd_rn(v, bias);
  if (flags & FM_EPI_RES_ADD) v = __fadd_rn(res, v);
  if (flags & FM_EPI_RES_SCALE) v = __fadd_rn(res, __fmul_rn(scale, v));
  if (flags & FM_EPI_ELU) v = fm_elu(v);
  if (flags & FM_EPI_GELU) v = fm_gelu(v);
  return v;
}

// Epilogue for one output element (generic kernel and split-K reduction).
FM_DEVICE void store_out(float acc, long m, int n, const GemmArgs& p) {
  const float bias = p.bias ? p.bias[n % p.bias_len] : 0.0f;
  const float scale = (p.flags & FM_EPI_RES_SCALE) ? p.scale[n] : 0.0f;
  const float res = (p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE)) ? p.res[m * p.N + n] : 0.0f;
  const float v = epilogue_v(acc, bias, res, scale, p.flags);
  if (p.y_rows == p.rows) {
    p.y[m * p.N + n] = v;
  } else {
    const int b = (int)(m / p.rows);
    const int t = (int)(m - (long)b * p.rows);
    if (t < p.y_rows) p.y[((long)b * p.y_rows + t) * p.N + n] = v;
  }
}

// Block -> tile.  Blocks are dispatched round-robin over the 8 XCDs (block b
// to XCD b % 8), each with its own L2; XCD x is given one contiguous range of
// tile indices (the first nb % 8 XCDs one tile more), so a row band's column
// tiles, which re-read the same input rows, share an L2.
FM_DEVICE int tile_index() {
  const int nb = gridDim.x;
  const int b = blockIdx.x;
  const int x = b % 8, q = nb / 8, r = nb % 8;
  return (x < r ? x * (q + 1) : r * (q + 1) + (x - r) * q) + b / 8;
}

// ---------------------------------------------------------------------------
// Fast kernel.  WK > 1: the waves form WK groups of WM*WN waves; group g takes
// k-tiles g, g + WK, ... and the groups' accumulators are summed in order.
template <int BM, int BN, int WM, int WN, int WK, int BK>
__global__ __launch_bounds__(NTHREADS) void gemm_fast_kernel(GemmArgs p) {
  static_assert(64 * WM * WN * WK == NTHREADS, "256 threads per block");
  constexpr int GT = 64 * WM * WN;  // threads per k-group
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int P = BK + 4;             // LDS row pitch (floats)
  constexpr int CPR = BK / 4;            // float4 chunks per tile row
  constexpr int HK = BK / 2;             // k values per MFMA lane half
  constexpr int APT = BM * BK / 4 / GT;  // float4 A chunks per thread per k-tile
  constexpr int BPT = BN * BK / 4 / GT;
  constexpr int STAGE = (BM + BN) * P;   // floats per stage
  static_assert(APT >= 1 && BPT >= 1 && APT * GT * 4 == BM * BK && BPT * GT * 4 == BN * BK, "tiling");
  static_assert(WK == 1 || 2 * STAGE * WK >= (WK - 1) * BM * BN, "LDS reduction fits the stages");

  __shared__ __attribute__((aligned(16))) float smem[2 * STAGE * WK];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int group = wave / (WM * WN);
  const int gtid = tid - group * GT;
  const int gwave = wave - group * WM * WN;
  const int wm0 = (gwave / WN) * WTM;
  const int wn0 = (gwave % WN) * WTN;
  float* gsm = smem + group * 2 * STAGE;

  const long M = (long)p.batch * p.rows;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = tile_index();
  const long m0 = (long)(tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;
  const int k_begin = blockIdx.y * p.k_split;
  const int k_end = min(p.K, k_begin + p.k_split);
  const bool replicate = p.flags & FM_REPLICATE;
  const bool tap_uniform = (p.C_in % BK) == 0;  // a k-tile never straddles two positions

  // Chunk c of a tile: row c / CPR, k offset 4 * (c % CPR).
  const int ck = (gtid % CPR) * 4;
  const float* a_base[APT];  // x + (b*L + p0) * C_in (valid rows), else null
  int a_p0[APT], a_bL[APT];
#pragma unroll
  for (int i = 0; i < APT; ++i) {
    const long m = m0 + gtid / CPR + i * (GT / CPR);
    a_base[i] = nullptr;
    a_p0[i] = 0;
    a_bL[i] = 0;
    if (m < M) {
      const int b = (int)(m / p.rows);
      const int t = (int)(m - (long)b * p.rows);
      a_p0[i] = t * p.rs - p.padL;
      a_bL[i] = b * p.L_in;
      a_base[i] = p.x + ((long)b * p.L_in + a_p0[i]) * p.C_in;
    }
  }
  const float* b_base[BPT];
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    const int n = n0 + gtid / CPR + i * (GT / CPR);
    b_base[i] = n < p.N ? p.w + (long)n * p.K : nullptr;
  }

  floatx4 ra[APT], rb[BPT];
  auto load = [&](int k0) {
    const int kg = k0 + ck;
    const bool kok = kg < k_end;
    const int tap = tap_uniform ? k0 / p.C_in : kg / p.C_in;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      ra[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (a_base[i] && kok) {
        int pos = a_p0[i] + tap;
        if (replicate) {
          pos = min(max(pos, 0), p.L_in - 1);
          ra[i] = *reinterpret_cast<const floatx4*>(p.x + ((long)a_bL[i] + pos) * p.C_in + (kg % p.C_in));
        } else if (pos >= 0 && pos < p.L_in) {
          ra[i] = *reinterpret_cast<const floatx4*>(a_base[i] + kg);
        }
      }
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      rb[i] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (b_base[i] && kok) rb[i] = *reinterpret_cast<const floatx4*>(b_base[i] + kg);
    }
  };
  auto store = [&](int stage) {
    float* As = gsm + stage * STAGE;
    float* Bs = As + BM * P;
    const bool elu = p.flags & FM_ELU_IN;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      floatx4 v = ra[i];
      if (elu) v = floatx4{fm_elu(v.x), fm_elu(v.y), fm_elu(v.z), fm_elu(v.w)};
      *reinterpret_cast<floatx4*>(As + (gtid / CPR + i * (GT / CPR)) * P + ck) = v;
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i)
      *reinterpret_cast<floatx4*>(Bs + (gtid / CPR + i * (GT / CPR)) * P + ck) = rb[i];
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int h = lane >> 5;
  const int lcol = lane & 31;
  const int ktiles = (k_end - k_begin + BK - 1) / BK;
  const int rounds = (ktiles + WK - 1) / WK;
  int kq = k_begin + group * BK;
  if (rounds > 0) {
    load(kq);
    store(0);
  }
  for (int q = 0; q < rounds; ++q) {
    const int cur = q & 1;
    __syncthreads();  // stage `cur` is complete; stage `cur ^ 1` is free
    const int knext = kq + WK * BK;
    if (q + 1 < rounds) load(knext);
    if (kq < k_end) {
      const float* As = gsm + cur * STAGE;
      const float* Bs = As + BM * P;
#pragma unroll
      for (int s4 = 0; s4 < BK / 8; ++s4) {
        floatx4 a[FM], b[FN];
#pragma unroll
        for (int i = 0; i < FM; ++i)
          a[i] = *reinterpret_cast<const floatx4*>(As + (wm0 + i * 32 + lcol) * P + h * HK + s4 * 4);
#pragma unroll
        for (int j = 0; j < FN; ++j)
          b[j] = *reinterpret_cast<const floatx4*>(Bs + (wn0 + j * 32 + lcol) * P + h * HK + s4 * 4);
#pragma unroll
        for (int e = 0; e < 4; ++e)
#pragma unroll
          for (int i = 0; i < FM; ++i)
#pragma unroll
            for (int j = 0; j < FN; ++j) acc[i][j] = fm_mfma32(a[i][e], b[j][e], acc[i][j]);
      }
    }
    if (q + 1 < rounds) store(cur ^ 1);
    kq = knext;
  }

  if constexpr (WK > 1) {
    // Groups 1..WK-1 park their tiles in LDS; group 0 adds them in order.
    __syncthreads();
    if (group > 0) {
      float* red = smem + (group - 1) * BM * BN;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            red[(wm0 + i * 32 + fm_mfma32_row(r, lane)) * BN + wn0 + j * 32 + lcol] = acc[i][j][r];
    }
    __syncthreads();
    if (group > 0) return;
#pragma unroll
    for (int g = 1; g < WK; ++g) {
      const float* red = smem + (g - 1) * BM * BN;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            acc[i][j][r] = __fadd_rn(acc[i][j][r],
                                     red[(wm0 + i * 32 + fm_mfma32_row(r, lane)) * BN + wn0 + j * 32 + lcol]);
    }
  }

  if (p.partial) {
    float* dst = p.partial + (long)blockIdx.y * M * p.N;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int n = n0 + wn0 + j * 32 + lcol;
      if (n >= p.N) continue;
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const long m = m0 + wm0 + i * 32 + fm_mfma32_row(r, lane);
          if (m < M) dst[m * p.N + n] = acc[i][j][r];
        }
    }
    return;
  }
  const bool crop = p.y_rows != p.rows;
  const bool has_res = p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE);
  // Residual loads first (all in flight together), then compute and store.
  float rv[FN][FM][16];
#pragma unroll
  for (int j = 0; j < FN; ++j)
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        rv[j][i][r] = 0.0f;
        if (has_res) {
          const long m = min(m0 + wm0 + i * 32 + fm_mfma32_row(r, lane), M - 1);
          const int n = min(n0 + wn0 + j * 32 + lcol, p.N - 1);
          rv[j][i][r] = p.res[m * p.N + n];
        }
      }
#pragma unroll
  for (int j = 0; j < FN; ++j) {
    const int n = n0 + wn0 + j * 32 + lcol;
    const int nc = min(n, p.N - 1);
    const float bias = p.bias ? p.bias[nc % p.bias_len] : 0.0f;
    const float scale = (p.flags & FM_EPI_RES_SCALE) ? p.scale[nc] : 0.0f;
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const long m = m0 + wm0 + i * 32 + fm_mfma32_row(r, lane);
        const float v = epilogue_v(acc[i][j][r], bias, rv[j][i][r], scale, p.flags);
        if (m >= M || n >= p.N) continue;
        if (!crop) {
          p.y[m * p.N + n] = v;
        } else {
          const int b = (int)(m / p.rows);
          const int t = (int)(m - (long)b * p.rows);
          if (t < p.y_rows) p.y[((long)b * p.y_rows + t) * p.N + n] = v;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Large-tile kernel: BK = 32, 8 waves of (BM/WM)x(BN/WN) outputs, each wave
// 64x32 (two 32x32 accumulators).  Used as 256x64 with one LDS stage refilled
// from a one-k-tile register prefetch (two barriers per k-tile), and as
// 128x128 with two LDS stages (one barrier per k-tile; the next k-tile's loads
// land in the other stage after the MFMAs).  Both stay near 100 VGPRs and
// under 80 KB of LDS, so two blocks share a CU and one block's barrier/store
// phase overlaps the other's MFMAs.  The 128x128 form measured 3-4% faster
// wherever N >= 128.  Loads are branch-free (clamped address plus a select)
// so the in-order instruction stream stays short.
// (lds_barrier, the LDS-only block barrier, lives in fm_common.h.)

// Sixteen zero bytes: the source of every out-of-window operand load in the
// zero-page loader (referenced from device code only).
__device__ __attribute__((aligned(16))) float g_zero16[4];

// ZP (zero padding and C_in a multiple of BK): a k-tile lies in one tap, so
// the tap comes from the uniform k0 (no per-lane division), each A row reads
// at its window start + k, and loads outside the window, past K or past N
// read g_zero16 instead of being masked after the load: about a third fewer
// VALU instructions per k-tile, which on this part do not overlap the MFMAs.
template <int BM, int BN, int WM, int WN, bool DB, bool ZP = false>
__global__ __launch_bounds__(64 * WM * WN) void gemm_big_kernel(GemmArgs p) {
  constexpr int NTH = 64 * WM * WN;
  constexpr int BK = 32, P = BK + 4, CPR = BK / 4, HK = BK / 2;
  constexpr int WTM = BM / WM, WTN = BN / WN;
  constexpr int FM = WTM / 32, FN = WTN / 32;
  constexpr int RPP = NTH / CPR;               // tile rows covered per pass
  constexpr int APT = BM / RPP, BPT = BN / RPP;
  static_assert(FM >= 1 && FN >= 1 && BPT >= 1 && APT * RPP == BM && BPT * RPP == BN, "tiling");

  // The operand stage(s) and, after the k-loop, the finished output tile share one array.
  constexpr int PC = BN + 4, NST = DB ? 2 : 1;
  constexpr int STAGE_F = (BM + BN) * P, TILE_F = BM * PC;
  __shared__ __attribute__((aligned(16))) float smem[NST * STAGE_F > TILE_F ? NST * STAGE_F : TILE_F];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm0 = (wave / WN) * WTM, wn0 = (wave % WN) * WTN;
  const long M = (long)p.batch * p.rows;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = tile_index();
  const long m0 = (long)(tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;
  const int k_begin = blockIdx.y * p.k_split;
  const int k_end = min(p.K, k_begin + p.k_split);
  const bool replicate = p.flags & FM_REPLICATE;
  const bool tap_uniform = (p.C_in % BK) == 0;
  const int ck = (tid % CPR) * 4;
  const int rrow = tid / CPR;

  // Per-row window origin: element offset of position p0 of batch b, p0 and
  // b*L.  Rows past M get p0 = INT_MIN / 2 so every position test fails.
  long a_org[APT];
  int a_p0[APT], a_bL[APT];
  const float* a_row[APT];  // ZP: the row's window start (tap 0)
#pragma unroll
  for (int i = 0; i < APT; ++i) {
    const int m = (int)min(m0 + rrow + i * RPP, M - 1);  // M < 2^31 (checked at launch)
    const int b = m / p.rows;
    const int t = m - b * p.rows;
    a_p0[i] = (m0 + rrow + i * RPP < M) ? t * p.rs - p.padL : INT_MIN / 2;
    a_bL[i] = b * p.L_in;
    a_org[i] = (long)b * p.L_in * p.C_in;
    a_row[i] = p.x + a_org[i] + (long)a_p0[i] * p.C_in;
  }
  int b_n[BPT];
  const float* b_row[BPT];  // ZP: weight row, null past N
#pragma unroll
  for (int i = 0; i < BPT; ++i) {
    b_n[i] = n0 + rrow + i * RPP;
    b_row[i] = b_n[i] < p.N ? p.w + (long)b_n[i] * p.K : nullptr;
  }

  // Prefetched rows stay raw in registers, with a validity mask; the zeroing
  // select happens at the LDS store, so nothing waits on the loads until the
  // next k-tile (a select right after the load would expose their latency).
  floatx4 ra[APT], rb[BPT];
  unsigned amask = 0, bmask = 0;
  auto load = [&](int k0) {
    if constexpr (ZP) {
      const int kg = k0 + ck;
      const bool kok = kg < k_end;
      const int tap = k0 / p.C_in;  // uniform
#pragma unroll
      for (int i = 0; i < APT; ++i) {
        const bool ok = kok & ((unsigned)(a_p0[i] + tap) < (unsigned)p.L_in);
        ra[i] = *reinterpret_cast<const floatx4*>(ok ? a_row[i] + kg : g_zero16);
      }
#pragma unroll
      for (int i = 0; i < BPT; ++i) {
        const bool ok = kok & (b_row[i] != nullptr);
        rb[i] = *reinterpret_cast<const floatx4*>(ok ? b_row[i] + kg : g_zero16);
      }
      return;
    }
    const int kg = k0 + ck;
    const bool kok = kg < k_end;
    const int kc = min(kg, p.K - 4);
    const int tap = tap_uniform ? k0 / p.C_in : kc / p.C_in;
    const int cin = kc - tap * p.C_in;  // channel within the position
    amask = bmask = 0;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int pos = a_p0[i] + tap;
      const bool ok = kok && (replicate ? a_p0[i] > INT_MIN / 2 : (pos >= 0 && pos < p.L_in));
      const int pc = min(max(pos, 0), p.L_in - 1);
      ra[i] = *reinterpret_cast<const floatx4*>(p.x + a_org[i] + (long)pc * p.C_in + cin);
      amask |= (unsigned)ok << i;
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const bool ok = kok && b_n[i] < p.N;
      rb[i] = *reinterpret_cast<const floatx4*>(p.w + (long)min(b_n[i], p.N - 1) * p.K + kc);
      bmask |= (unsigned)ok << i;
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int h = lane >> 5, lcol = lane & 31;
  const bool elu_in = p.flags & FM_ELU_IN;
  auto store = [&](int stage) {
    float* As = smem + stage * STAGE_F;
    float* Bs = As + BM * P;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      floatx4 v = (ZP || ((amask >> i) & 1)) ? ra[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (elu_in) v = floatx4{fm_elu(v.x), fm_elu(v.y), fm_elu(v.z), fm_elu(v.w)};
      *reinterpret_cast<floatx4*>(As + (rrow + i * RPP) * P + ck) = v;
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i)
      *reinterpret_cast<floatx4*>(Bs + (rrow + i * RPP) * P + ck) =
          (ZP || ((bmask >> i) & 1)) ? rb[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  };
  auto mma = [&](int stage) {
    const float* As = smem + stage * STAGE_F;
    const float* Bs = As + BM * P;
#pragma unroll
    for (int s4 = 0; s4 < BK / 8; ++s4) {
      floatx4 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i)
        a[i] = *reinterpret_cast<const floatx4*>(As + (wm0 + i * 32 + lcol) * P + h * HK + s4 * 4);
#pragma unroll
      for (int j = 0; j < FN; ++j)
        b[j] = *reinterpret_cast<const floatx4*>(Bs + (wn0 + j * 32 + lcol) * P + h * HK + s4 * 4);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = fm_mfma32(a[i][e], b[j][e], acc[i][j]);
    }
  };
  if constexpr (DB) {
    if (k_begin < k_end) {
      load(k_begin);
      store(0);
    }
    __syncthreads();
    int cur = 0;
    for (int k0 = k_begin; k0 < k_end; k0 += BK) {
      const bool more = k0 + BK < k_end;
      if (more) load(k0 + BK);
      mma(cur);
      if (more) store(cur ^ 1);
      __syncthreads();  // stage `cur` is free, stage `cur ^ 1` is complete
      cur ^= 1;
    }
  } else {
    if (k_begin < k_end) load(k_begin);
    for (int k0 = k_begin; k0 < k_end; k0 += BK) {
      __syncthreads();
      store(0);
      __syncthreads();
      if (k0 + BK < k_end) load(k0 + BK);
      mma(0);
    }
    __syncthreads();  // every wave is done reading the operand stage
  }

  // Epilogue through LDS: the waves drop their accumulators into the tile,
  // then each thread finishes float4 runs of a row (bias, residual, ELU) with
  // one bounds check per run and 16-byte loads and stores.
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r)
        smem[(wm0 + i * 32 + fm_mfma32_row(r, lane)) * PC + wn0 + j * 32 + lcol] = acc[i][j][r];
  __syncthreads();
  // A thread's runs share one column group (NTH is a multiple of BN / 4), so
  // bias and scale load once; the LDS reads and residual loads of all runs
  // are issued before the first store.
  const bool crop = p.y_rows != p.rows;
  const bool has_res = p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE);
  float* part = p.partial ? p.partial + (long)blockIdx.y * M * p.N : nullptr;
  constexpr int CG = BN / 4, RSTEP = NTH / CG, NRUN = BM / RSTEP;
  static_assert(NTH % CG == 0 && BM % RSTEP == 0, "epilogue runs");
  const int c = (tid % CG) * 4, r0 = tid / CG;
  const int n = n0 + c;
  const bool n_ok = n < p.N;
  const int ncl = n_ok ? n : 0;
  const floatx4 bias = (p.bias && !part) ? *reinterpret_cast<const floatx4*>(p.bias + ncl % p.bias_len)
                                         : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const floatx4 scale = ((p.flags & FM_EPI_RES_SCALE) && !part)
                            ? *reinterpret_cast<const floatx4*>(p.scale + ncl)
                            : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  floatx4 v[NRUN], res[NRUN];
#pragma unroll
  for (int u = 0; u < NRUN; ++u) {
    const int r = r0 + u * RSTEP;
    const long m = min(m0 + r, M - 1);
    v[u] = *reinterpret_cast<const floatx4*>(smem + r * PC + c);
    res[u] = (has_res && !part) ? *reinterpret_cast<const floatx4*>(p.res + m * p.N + ncl)
                                : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  }
#pragma unroll
  for (int u = 0; u < NRUN; ++u) {
    const long m = m0 + r0 + u * RSTEP;
    if (m >= M || !n_ok) continue;
    if (part) {
      *reinterpret_cast<floatx4*>(part + m * p.N + n) = v[u];
      continue;
    }
    floatx4 o = v[u];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = epilogue_v(o[e], bias[e], res[u][e], scale[e], p.flags);
    long dst = m * p.N + n;
    if (crop) {
      const int b = (int)(m / p.rows);
      const int t = (int)(m - (long)b * p.rows);
      if (t >= p.y_rows) continue;
      dst = ((long)b * p.y_rows + t) * p.N + n;
    }
    *reinterpret_cast<floatx4*>(p.y + dst) = o;
  }
}

// ---------------------------------------------------------------------------
// Direct-load kernel: the operand tiles travel from global memory straight
// into LDS (global_load_lds_dwordx4, one 16-byte chunk per lane, written at
// lane * 16 bytes of the wave's 1 KB window), so the k-loop holds no prefetch
// registers and issues no vector instructions to stage operands.  An NST-deep
// LDS ring of BK-deep k-tiles is refilled NST - 1 k-tiles ahead, with one
// barrier per k-tile (the shipped tiles: two stages, BK = 32, or BK = 64 for
// the one-block-per-CU 64x128 tile; BK = 16 with three stages measured
// slower).  Each lane picks the global chunk that
// belongs in its LDS slot: slot (row r, position cp) holds chunk
// cp ^ ((r / SWR) % CPR) of row r, so the MFMA fragment reads (eight rows per
// 16-byte read phase) spread over all 64 banks.  Loads that fall outside the
// input window, past M or past N read the zero page g_zero16.
// Requirements: zero padding, no ELU on load, C_in, K and the K-split
// boundaries multiples of BK (run_gemm guarantees them).  8 waves as
// 2 x WN; the epilogue runs in two halves of BM / 2 rows (one wave row each)
// so that the output tile fits in the ring's LDS: 64 KB at 128 x 128, two
// blocks per CU.
template <int BM, int BN, int WN, int BK, int NST, int WPE>
__global__ __launch_bounds__(512) __attribute__((amdgpu_waves_per_eu(WPE, WPE))) void gemm_dl_kernel(GemmArgs p) {
  constexpr int NTH = 512, WM = 2;
  static_assert((BK == 16 || BK == 32 || BK == 64) && (NST == 2 || NST == 3), "ring shape");
  constexpr int CPR = BK / 4, RPI = 64 / CPR;  // chunks per row, rows per load instruction
  constexpr int SWR = 64 / BK;                 // rows per full sweep of the 64 banks
  static_assert(WM * WN == 8, "eight waves");
  constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32;
  constexpr int AI = BM / (8 * RPI), BI = BN / (8 * RPI);  // load instructions per wave per stage
  static_assert(FM >= 1 && FN >= 1 && AI >= 1 && BI >= 1 && AI * 8 * RPI == BM && BI * 8 * RPI == BN, "tiling");
  constexpr int LPS = AI + BI;
  constexpr int STAGE_F = (BM + BN) * BK;
  constexpr int HM = BM / 2, PC = BN + 4, TILE_F = HM * PC;
  __shared__ __attribute__((aligned(16))) float smem[NST * STAGE_F > TILE_F ? NST * STAGE_F : TILE_F];

  // The wave index is uniform: LDS window addresses stay in scalar registers.
  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave / WN;
  const int wm0 = wr * WTM, wn0 = (wave % WN) * WTN;
  const long M = (long)p.batch * p.rows;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = tile_index();
  const long m0 = (long)(tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;
  const int k_begin = blockIdx.y * p.k_split;
  const int k_end = min(p.K, k_begin + p.k_split);

  // This lane's chunk of each load instruction: tile row lr + 16 * (instr),
  // chunk position cp within the row, global chunk cg.
  const int lr = lane / CPR, cp = lane % CPR;
  const float* a_row[AI];
  int a_p0[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int r = (wave * AI + i) * RPI + lr;
    const long mm = m0 + r;
    const int m = (int)min(mm, M - 1);
    const int b = (int)fm_div((unsigned)m, p.rows_div);
    const int t = m - b * p.rows;
    a_p0[i] = mm < M ? t * p.rs - p.padL : INT_MIN / 2;
    a_row[i] = p.x + (long)b * p.L_in * p.C_in + (long)a_p0[i] * p.C_in + 4 * (cp ^ ((r / SWR) & (CPR - 1)));
  }
  const float* b_row[BI];
#pragma unroll
  for (int i = 0; i < BI; ++i) {
    const int r = (wave * BI + i) * RPI + lr;
    const int n = n0 + r;
    b_row[i] = n < p.N ? p.w + (long)n * p.K + 4 * (cp ^ ((r / SWR) & (CPR - 1))) : nullptr;
  }
  auto issue = [&](int stage, int k0) {
    float* As = smem + stage * STAGE_F;
    float* Bs = As + BM * BK;
    const int tap = k0 / p.C_in;  // uniform: a k-tile lies in one tap
#pragma unroll
    for (int i = 0; i < AI; ++i) {
      const bool ok = (unsigned)(a_p0[i] + tap) < (unsigned)p.L_in;
      const float* src = ok ? a_row[i] + k0 : g_zero16;
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(As + (wave * AI + i) * RPI * BK),
                                       16, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < BI; ++i) {
      const float* src = b_row[i] ? b_row[i] + k0 : g_zero16;
      __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)src,
                                       (__attribute__((address_space(3))) void*)(Bs + (wave * BI + i) * RPI * BK),
                                       16, 0, 0);
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int h = lane >> 5, lcol = lane & 31;
  const int nkt = (k_end - k_begin) / BK;
  if (nkt > 0) issue(0, k_begin);
  if (NST == 3 && nkt > 1) issue(1, k_begin + BK);
  for (int kt = 0; kt < nkt; ++kt) {
    // This lane's loads of stage kt are done once at most the next stage's remain.
    if (NST == 3 && kt + 1 < nkt) asm volatile("s_waitcnt vmcnt(%0)" ::"n"(LPS) : "memory");
    else asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    // Every wave's loads of stage kt landed, and every wave's reads of stage
    // (kt + 2) % 3 completed (their values fed the previous MFMAs).  A bare
    // s_barrier: __syncthreads would also wait for the stage kt + 1 loads.
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + NST - 1 < nkt) issue((kt + NST - 1) % NST, k_begin + (kt + NST - 1) * BK);
    const float* As = smem + (kt % NST) * STAGE_F;
    const float* Bs = As + BM * BK;
#pragma unroll
    for (int q = 0; q < BK / 8; ++q) {
      const int c = (BK / 8) * h + q;  // k = (BK / 2) h + 4q + e at MFMA step 4q + e
      floatx4 a[FM], b[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm0 + i * 32 + lcol;
        a[i] = *reinterpret_cast<const floatx4*>(As + row * BK + 4 * (c ^ ((row / SWR) & (CPR - 1))));
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const int row = wn0 + j * 32 + lcol;
        b[j] = *reinterpret_cast<const floatx4*>(Bs + row * BK + 4 * (c ^ ((row / SWR) & (CPR - 1))));
      }
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < FM; ++i)
#pragma unroll
          for (int j = 0; j < FN; ++j) acc[i][j] = fm_mfma32(a[i][e], b[j][e], acc[i][j]);
    }
  }
  // Every wave is done reading the ring.  The epilogue's barriers order LDS
  // traffic only: __syncthreads would also wait for the previous half's
  // global stores to complete, serialising the two halves' HBM writes.
  lds_barrier();

  const bool crop = p.y_rows != p.rows;
  const bool has_res = p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE);
  float* part = p.partial ? p.partial + (long)blockIdx.y * M * p.N : nullptr;
  constexpr int CG = BN / 4, RSTEP = NTH / CG, NRUN = HM / RSTEP, RB = WPE > 4 ? 1 : (NRUN < 2 ? NRUN : 2);
  static_assert(NTH % CG == 0 && HM % RSTEP == 0 && NRUN % RB == 0, "epilogue runs");
  const int c = (tid % CG) * 4, r0 = tid / CG;
  const int n = n0 + c;
  const bool n_ok = n < p.N;
  const int ncl = n_ok ? n : 0;
  const floatx4 bias = (p.bias && !part) ? *reinterpret_cast<const floatx4*>(p.bias + ncl % p.bias_len)
                                         : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  const floatx4 scale = ((p.flags & FM_EPI_RES_SCALE) && !part)
                            ? *reinterpret_cast<const floatx4*>(p.scale + ncl)
                            : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int hf = 0; hf < 2; ++hf) {
    if (wr == hf) {
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r)
            smem[(i * 32 + fm_mfma32_row(r, lane)) * PC + wn0 + j * 32 + lcol] = acc[i][j][r];
    }
    lds_barrier();
    const long mh = m0 + hf * HM;
#pragma unroll
    for (int u0 = 0; u0 < NRUN; u0 += RB) {
      floatx4 v[RB], res[RB];
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const int r = r0 + (u0 + u) * RSTEP;
        const long m = min(mh + r, M - 1);
        v[u] = *reinterpret_cast<const floatx4*>(smem + r * PC + c);
        res[u] = (has_res && !part) ? *reinterpret_cast<const floatx4*>(p.res + m * p.N + ncl)
                                    : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      }
#pragma unroll
      for (int u = 0; u < RB; ++u) {
        const long m = mh + r0 + (u0 + u) * RSTEP;
        if (m >= M || !n_ok) continue;
        if (part) {
          *reinterpret_cast<floatx4*>(part + m * p.N + n) = v[u];
          continue;
        }
        floatx4 o = v[u];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = epilogue_v(o[e], bias[e], res[u][e], scale[e], p.flags);
        long dst = m * p.N + n;
        if (crop) {
          const int b = (int)(m / p.rows);
          const int t = (int)(m - (long)b * p.rows);
          if (t >= p.y_rows) continue;
          dst = ((long)b * p.y_rows + t) * p.N + n;
        }
        *reinterpret_cast<floatx4*>(p.y + dst) = o;
      }
    }
    if (hf == 0) lds_barrier();  // the half tile is consumed before the next half lands
  }
}

// ---------------------------------------------------------------------------
// Mid-size kernel for few-row / long-K contractions: BM x BN in {32, 64}^2,
// 4 waves, each owning a 32x32 output tile as 2x2 independent 16x16x4 FP32
// MFMA chains; the waves form (BM/32) x (BN/32) x WK groups, and with WK > 1
// the groups split every k-tile and their tiles are summed through LDS in
// group order.  k-tile BK = 128 staged in one LDS stage (row pitch BK + 4),
// refilled from a one-k-tile register prefetch, so each barrier pair
// brackets 128 / WK MFMAs per wave.  Lane (g = l/16, i = l%16) carries k =
// 32g + 4t + e of the k-tile at MFMA step 4t+e: 16-byte LDS reads.
FM_DEVICE floatx4 fm_mfma16x4(float a, float b, floatx4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

template <int BM, int BN, int WK>
__global__ __launch_bounds__(256) void gemm_mid_kernel(GemmArgs p) {
  constexpr int NTH = 256, BK = 128, P = BK + 4, CPR = BK / 4;
  constexpr int WMN = BN / 32;                   // waves along N within a k-group
  static_assert((BM / 32) * (BN / 32) * WK == 4, "4 waves");
  constexpr int RPP = NTH / CPR;                 // rows per load pass (8)
  constexpr int APT = BM / RPP, BPT = BN / RPP;
  constexpr int KSL = BK / WK;                   // k per group per k-tile
  constexpr int TSTEPS = KSL / 16;               // float4 steps of the group's slice per lane group
  constexpr int STAGE = (BM + BN) * P;
  constexpr int RED = (WK - 1) * BM * (BN + 4);
  __shared__ __attribute__((aligned(16))) float msm[STAGE > RED ? STAGE : RED];
  float* As = msm;
  float* Bs = msm + BM * P;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int grp = wave / ((BM / 32) * WMN);
  const int wv = wave % ((BM / 32) * WMN);
  const int wm0 = (wv / WMN) * 32, wn0 = (wv % WMN) * 32;
  const int g = lane >> 4, li = lane & 15;
  const long M = (long)p.batch * p.rows;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = tile_index();
  const long m0 = (long)(tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;
  const int k_begin = blockIdx.y * p.k_split;
  const int k_end = min(p.K, k_begin + p.k_split);
  const bool replicate = p.flags & FM_REPLICATE;
  const int ck = (tid % CPR) * 4;
  const int rrow = tid / CPR;

  long a_org[APT];
  int a_p0[APT];
#pragma unroll
  for (int i = 0; i < APT; ++i) {
    const long m = min(m0 + rrow + i * RPP, M - 1);
    const int b = (int)(m / p.rows);
    const int t = (int)(m - (long)b * p.rows);
    a_p0[i] = (m0 + rrow + i * RPP < M) ? t * p.rs - p.padL : INT_MIN / 2;
    a_org[i] = (long)b * p.L_in * p.C_in;
  }
  floatx4 ra[APT], rb[BPT];
  unsigned amask = 0, bmask = 0;
  auto load = [&](int k0) {
    const int kg = k0 + ck;
    const bool kok = kg < k_end;
    const int kc = min(kg, p.K - 4);
    const int tap = kc / p.C_in;
    const int cin = kc - tap * p.C_in;
    amask = bmask = 0;
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      const int pos = a_p0[i] + tap;
      const bool ok = kok && (replicate ? a_p0[i] > INT_MIN / 2 : (pos >= 0 && pos < p.L_in));
      const int pc = min(max(pos, 0), p.L_in - 1);
      ra[i] = *reinterpret_cast<const floatx4*>(p.x + a_org[i] + (long)pc * p.C_in + cin);
      amask |= (unsigned)ok << i;
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i) {
      const int n = n0 + rrow + i * RPP;
      const bool ok = kok && n < p.N;
      rb[i] = *reinterpret_cast<const floatx4*>(p.w + (long)min(n, p.N - 1) * p.K + kc);
      bmask |= (unsigned)ok << i;
    }
  };
  const bool elu_in = p.flags & FM_ELU_IN;

  floatx4 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i)
#pragma unroll
    for (int j = 0; j < 2; ++j) acc[i][j] = floatx4{0.0f, 0.0f, 0.0f, 0.0f};

  const int kbase = grp * KSL;  // this group's k offset within a k-tile
  if (k_begin < k_end) load(k_begin);
  for (int k0 = k_begin; k0 < k_end; k0 += BK) {
    __syncthreads();
#pragma unroll
    for (int i = 0; i < APT; ++i) {
      floatx4 v = ((amask >> i) & 1) ? ra[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
      if (elu_in) v = floatx4{fm_elu(v.x), fm_elu(v.y), fm_elu(v.z), fm_elu(v.w)};
      *reinterpret_cast<floatx4*>(As + (rrow + i * RPP) * P + ck) = v;
    }
#pragma unroll
    for (int i = 0; i < BPT; ++i)
      *reinterpret_cast<floatx4*>(Bs + (rrow + i * RPP) * P + ck) =
          ((bmask >> i) & 1) ? rb[i] : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
    __syncthreads();
    if (k0 + BK < k_end) load(k0 + BK);
#pragma unroll
    for (int t = 0; t < TSTEPS; ++t) {
      const int kk = kbase + (KSL / 4) * g + 4 * t;
      floatx4 a[2], b[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) a[i] = *reinterpret_cast<const floatx4*>(As + (wm0 + 16 * i + li) * P + kk);
#pragma unroll
      for (int j = 0; j < 2; ++j) b[j] = *reinterpret_cast<const floatx4*>(Bs + (wn0 + 16 * j + li) * P + kk);
#pragma unroll
      for (int e = 0; e < 4; ++e)
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
          for (int j = 0; j < 2; ++j) acc[i][j] = fm_mfma16x4(a[i][e], b[j][e], acc[i][j]);
    }
  }

  if constexpr (WK > 1) {
    constexpr int PRD = BN + 4;
    __syncthreads();
    if (grp > 0) {
      float* red = msm + (grp - 1) * BM * PRD;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r) red[(wm0 + 16 * i + 4 * g + r) * PRD + wn0 + 16 * j + li] = acc[i][j][r];
    }
    __syncthreads();
    if (grp > 0) return;
#pragma unroll
    for (int q = 1; q < WK; ++q) {
      const float* red = msm + (q - 1) * BM * PRD;
#pragma unroll
      for (int i = 0; i < 2; ++i)
#pragma unroll
        for (int j = 0; j < 2; ++j)
#pragma unroll
          for (int r = 0; r < 4; ++r)
            acc[i][j][r] = __fadd_rn(acc[i][j][r], red[(wm0 + 16 * i + 4 * g + r) * PRD + wn0 + 16 * j + li]);
    }
  }

  const bool crop = p.y_rows != p.rows;
  const bool has_res = p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE);
  float* part = p.partial ? p.partial + (long)blockIdx.y * M * p.N : nullptr;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int n = n0 + wn0 + 16 * j + li;
    const int nc = min(n, p.N - 1);
    const float bias = p.bias ? p.bias[nc % p.bias_len] : 0.0f;
    const float scale = (p.flags & FM_EPI_RES_SCALE) ? p.scale[nc] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const long m = m0 + wm0 + 16 * i + 4 * g + r;
        if (m >= M || n >= p.N) continue;
        if (part) {
          part[m * p.N + n] = acc[i][j][r];
          continue;
        }
        const float res = has_res ? p.res[m * p.N + n] : 0.0f;
        const float v = epilogue_v(acc[i][j][r], bias, res, scale, p.flags);
        if (!crop) {
          p.y[m * p.N + n] = v;
        } else {
          const int b = (int)(m / p.rows);
          const int t = (int)(m - (long)b * p.rows);
          if (t < p.y_rows) p.y[((long)b * p.y_rows + t) * p.N + n] = v;
        }
      }
  }
}

// ---------------------------------------------------------------------------
// Generic kernel: 64x64 tiles, one output element pair per thread per step,
// scalar loads.  Used only when C_in or K is not a multiple of 4.
__global__ __launch_bounds__(256) void gemm_generic_kernel(GemmArgs p) {
  constexpr int TM = 64, TN = 64, TK = 16;
  __shared__ float As[TK][TM + 1];
  __shared__ float Bs[TK][TN + 1];
  const long M = (long)p.batch * p.rows;
  const int tiles_n = (p.N + TN - 1) / TN;
  const long m0 = (long)(blockIdx.x / tiles_n) * TM;
  const int n0 = (blockIdx.x % tiles_n) * TN;
  const int k_begin = blockIdx.y * p.k_split;
  const int k_end = min(p.K, k_begin + p.k_split);
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;  // 16 x 16 threads, 4 x 4 outputs each
  float acc[4][4] = {};
  for (int k0 = k_begin; k0 < k_end; k0 += TK) {
    for (int e = threadIdx.x; e < TK * TM; e += 256) {
      const int r = e / TK, kk = e % TK;
      const long m = m0 + r;
      const int kg = k0 + kk;
      float v = 0.0f;
      if (m < M && kg < k_end) {
        const int b = (int)(m / p.rows);
        const int t = (int)(m - (long)b * p.rows);
        int pos = t * p.rs - p.padL + kg / p.C_in;
        bool ok = true;
        if (p.flags & FM_REPLICATE) pos = min(max(pos, 0), p.L_in - 1);
        else ok = pos >= 0 && pos < p.L_in;
        if (ok) v = p.x[((long)b * p.L_in + pos) * p.C_in + kg % p.C_in];
        if (p.flags & FM_ELU_IN) v = fm_elu(v);
      }
      As[kk][r] = v;
    }
    for (int e = threadIdx.x; e < TK * TN; e += 256) {
      const int c = e / TK, kk = e % TK;
      const int n = n0 + c, kg = k0 + kk;
      Bs[kk][c] = (n < p.N && kg < k_end) ? p.w[(long)n * p.K + kg] : 0.0f;
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < TK; ++kk)
#pragma unroll
      for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = fmaf(As[kk][ty + 16 * i], Bs[kk][tx + 16 * j], acc[i][j]);
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const long m = m0 + ty + 16 * i;
      const int n = n0 + tx + 16 * j;
      if (m >= M || n >= p.N) continue;
      if (p.partial)
        p.partial[((long)blockIdx.y * M + m) * p.N + n] = acc[i][j];
      else
        store_out(acc[i][j], m, n, p);
    }
}

// Sums global split-K partials in split order and applies the epilogue.
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

// Vector form (N and bias_len multiples of 4, fewer than 2^31 float4s): each
// thread sums four adjacent outputs of one row over the splits, in split
// order as above, and applies the same epilogue; its row comes from a
// magic-number division instead of a 64-bit one per element.
__global__ __launch_bounds__(256) void splitk_reduce4_kernel(GemmArgs p, int splits, FmDivisor n4_div) {
  const long M = (long)p.batch * p.rows;
  const long total = M * p.N;
  const unsigned total4 = (unsigned)(total / 4);
  const int N4 = p.N / 4;
  const bool res_in = p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE);
  const bool crop = p.y_rows != p.rows;
  for (unsigned e4 = blockIdx.x * blockDim.x + threadIdx.x; e4 < total4; e4 += gridDim.x * blockDim.x) {
    const long e = 4L * e4;
    floatx4 s = *reinterpret_cast<const floatx4*>(p.partial + e);
    for (int k = 1; k < splits; ++k) {
      const floatx4 q = *reinterpret_cast<const floatx4*>(p.partial + (long)k * total + e);
#pragma unroll
      for (int c = 0; c < 4; ++c) s[c] = __fadd_rn(s[c], q[c]);
    }
    const int m = (int)fm_div(e4, n4_div);
    const int n = 4 * ((int)e4 - m * N4);
    const floatx4 zero = {0.0f, 0.0f, 0.0f, 0.0f};
    const floatx4 bias = p.bias ? *reinterpret_cast<const floatx4*>(p.bias + n % p.bias_len) : zero;
    const floatx4 scale = (p.flags & FM_EPI_RES_SCALE) ? *reinterpret_cast<const floatx4*>(p.scale + n) : zero;
    const floatx4 res = res_in ? *reinterpret_cast<const floatx4*>(p.res + e) : zero;
#pragma unroll
    for (int c = 0; c < 4; ++c) s[c] = epilogue_v(s[c], bias[c], res[c], scale[c], p.flags);
    long dst = e;
    if (crop) {
      const int b = (int)fm_div((unsigned)m, p.rows_div);
      const int t = m - b * p.rows;
      if (t >= p.y_rows) continue;
      dst = ((long)b * p.y_rows + t) * p.N + n;
    }
    *reinterpret_cast<floatx4*>(p.y + dst) = s;
  }
}

// ---------------------------------------------------------------------------
// FP32 contraction on the bf16 matrix cores ("bf16x6").  Every FP32 operand
// is the sum of three round-to-nearest bf16 pieces, v = v0 + v1 + v2, exact to
// within 2^-24 |v| (each piece holds the next 8 significant bits of what the
// previous ones left).  A product a*b is then the six cross terms whose
// pieces' orders sum to at most 2 (a2b0 + a1b1 + a0b2 + a1b0 + a0b1 + a0b0,
// smallest first); the three dropped terms are below 2^-24 |a b|.  Each
// bf16 x bf16 product is exact in FP32 and the MFMA accumulates in FP32, so
// the result carries FP32 rounding error (measured against float64 on the
// SEANet shapes: rms 2-3e-7 of the output scale, as the FP32 MFMA path) while
// v_mfma_f32_32x32x16_bf16 delivers 16x the FP32 MFMA rate: six of them cost
// 0.375 of the FP32 instruction time per k.
// Weights are split once (fm_split_weights) into planes [3][K/16][N][16]
// stored right after the FP32 W^T; A tiles reach LDS as FP32 and each wave
// splits its own fragments (gemm_x6d_kernel below).  Measured against the
// FP32 direct-load tile on the SEANet shapes: 1.3-1.5x.
// W^T [N][K] fp32 -> three bf16 planes in k16-tile order [3][K/16][N][16]:
// the 16 k of one row are 32 contiguous bytes and the rows of a k-tile are
// adjacent, so 32 rows of one k-tile are one 1 KB run.
__global__ __launch_bounds__(256) void split_weights_kernel(const float* __restrict__ w, int N, int K,
                                                            bf16x4* __restrict__ out) {
  const long i = (long)blockIdx.x * 256 + threadIdx.x;  // float4 index into W^T
  const long n4 = (long)N * K / 4;
  if (i >= n4) return;
  const long n = 4 * i / K;
  const int k = (int)(4 * i - n * K);
  bf16x4 h0, h1, h2;
  split3(*reinterpret_cast<const floatx4*>(w + 4 * i), h0, h1, h2);
  const long o = (((long)(k >> 4) * N + n) * 16 + (k & 15)) / 4;
  out[o] = h0;
  out[n4 + o] = h1;
  out[2 * n4 + o] = h2;
}

// ---------------------------------------------------------------------------
// bf16x6 tile with the FP32 A operand loaded global -> LDS directly: each
// lane's 16-byte chunk of the 16-deep A k-tile lands in an XOR-swizzled slot
// (chunk c of row r at position c ^ ((r / 4) & 3), so the 16-lane groups of a
// fragment read hit distinct banks) with the zero page for out-of-window and
// past-M rows; the B planes travel global -> LDS directly too
// (global_load_lds_dwordx4; 32 rows of a k-tile are one contiguous 1 KB run
// of the k16-tile ordered planes, LDS rows of 32 bytes read as 1 KB
// fragments).  NST-stage ring, one barrier per k-tile.  Each wave splits its
// own A fragments after the LDS read, so no register staging or wait sits in
// the k-loop; a wave tile spanning the block's columns (WN = 1: 32 x 128)
// splits every A element once, narrower ones (32 x 64) twice.  Products in
// the order a1b1, a1b0, a0b1, a2b0, a0b2, a0b0 per k-tile.  The epilogue
// stores straight from the accumulators.  Tiles: 256 x 128 (eight waves of
// 32 x 128, 56 KB, two blocks per CU) where it gives at least 384 tiles;
// 128 x 128 / 64 x 128 / 192 x 128 (waves of 32 x 64) for smaller grids.
// Blocks per CU of the bf16x6 tiles, set explicitly (register budget below,
// LDS floor in the kernel), measured per tile on the C2-C4 shapes:
//   256x128: two (held to 128 VGPRs; at its natural 138 only one fits:
//            dec.up4 at C4 633 -> 411 us);
//   64x128: four (an LDS floor above 32 KB and 128 VGPRs; at three the
//            K-split shapes ran 14% slower);
//   192x128 with 16-deep k-tiles: one (an LDS floor above 80 KB; two per CU
//            ran the ELU-on-load form 13% slower);
//   128x128 of four 32x128 waves: three (an LDS floor above 40 KB and 168
//            VGPRs; four ran 9% slower);
//   the rest as their LDS ring and natural register use give.
constexpr int x6d_min_waves_per_simd(int BM, int NW, int WN) {
  if (BM == 256 && WN == 1) return 4;
  if (BM == 64) return 4;
  if (BM == 128 && WN == 1) return 3;
  return (NW + 3) / 4;  // what the block size implies (the compiler's default)
}
constexpr int x6d_lds_floor(int BM, int WN, int KS) {
  if (BM == 192 && KS == 1) return 80 * 1024 + 1024;
  if (BM == 128 && WN == 1) return 40 * 1024 + 1024;
  if (BM == 64) return 32 * 1024 + 1024;
  return 0;
}
template <int BM, int BN, int WM, int WN, int NST, bool ELU, int KS = 1>
__global__ __launch_bounds__(64 * WM * WN) __attribute__((amdgpu_waves_per_eu(x6d_min_waves_per_simd(BM, WM * WN, WN))))
void gemm_x6d_kernel(GemmArgs p, const __bf16* __restrict__ w3) {
  // KS 16-deep k sub-tiles per stage (BK = 16 KS), run in k order.
  constexpr int NW = WM * WN, NTH = 64 * NW, BK = 16 * KS;
  static_assert(NW % 2 == 0 && NW <= 12 && NST == 2, "two to twelve waves, two stages");
  constexpr int WTM = BM / WM, WTN = BN / WN, FM = WTM / 32, FN = WTN / 32;
  // A: 16-byte chunks per row, rows per load instruction, and the swizzle
  // period that gives 16 consecutive rows 16 distinct bank groups.
  constexpr int CPR = 4 * KS, RPI = 64 / CPR, SWR = 16 / CPR;
  constexpr int AI = BM / (NW * RPI);        // A load instructions per wave per stage
  static_assert(AI >= 1 && AI * NW * RPI == BM && FM >= 1 && FN >= 1 && BN % 32 == 0, "tiling");
  constexpr int PLANE_B = BN * BK * 2, STAGE_A = BM * BK * 4, STAGE = STAGE_A + 3 * PLANE_B;
  constexpr int NBI = 3 * KS * BN / 32;  // 1 KB B load instructions per stage
  constexpr int LDS = NST * STAGE > x6d_lds_floor(BM, WN, KS) ? NST * STAGE : x6d_lds_floor(BM, WN, KS);
  __shared__ __attribute__((aligned(16))) char smem[LDS];

  const int tid = threadIdx.x, lane = tid & 63, wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wr = wave / WN;
  const int wm0 = wr * WTM, wn0 = (wave % WN) * WTN;
  const long M = (long)p.batch * p.rows;
  const int tiles_n = (p.N + BN - 1) / BN;
  const int tile = tile_index();
  const long m0 = (long)(tile / tiles_n) * BM;
  const int n0 = (tile % tiles_n) * BN;
  const int k_begin = blockIdx.y * p.k_split;
  const int k_end = min(p.K, k_begin + p.k_split);

  // This lane's chunk of each A load instruction: tile row r, chunk position
  // cp (global chunk cp ^ swizzle).
  const int lr = lane / CPR, cp = lane % CPR;
  const float* a_row[AI];
  int a_p0[AI], a_voff[AI];
#pragma unroll
  for (int i = 0; i < AI; ++i) {
    const int r = (wave * AI + i) * RPI + lr;
    const long mm = m0 + r;
    const int m = (int)min(mm, M - 1);
    const int b = (int)fm_div((unsigned)m, p.rows_div);
    const int t = m - b * p.rows;
    a_p0[i] = mm < M ? t * p.rs - p.padL : INT_MIN / 2;
    a_row[i] = p.x + (long)b * p.L_in * p.C_in + (long)a_p0[i] * p.C_in + 4 * (cp ^ ((r / SWR) & (CPR - 1)));
    a_voff[i] = (int)((a_row[i] - p.x) * 4);
  }
  // Inputs below 2 GiB load A through a buffer resource too: per k-tile only
  // the window test and a select on a 32-bit offset (out-of-window and past-M
  // rows read out of range, i.e. zeros).
  const long x_bytes = (long)p.batch * p.L_in * p.C_in * 4;
  const bool a_buf = x_bytes < 0x7fffffffL;
  const __amdgpu_buffer_rsrc_t ra = fm_buffer(p.x, a_buf ? (int)x_bytes : 0);
  const long KN = (long)p.K * p.N;
  // B plane loads through a buffer resource over the three planes: lane
  // offsets computed once, out-of-range (past-N) lanes read zeros.
  constexpr int NBW = (NBI + NW - 1) / NW;  // B load instructions per wave (at most)
  const __amdgpu_buffer_rsrc_t rb = fm_buffer(w3, (int)(3 * KN * 2));
  int b_voff[NBW], b_lds[NBW];
#pragma unroll
  for (int q = 0; q < NBW; ++q) {
    const int i = min(wave + q * NW, NBI - 1);
    const int pl = i / (KS * BN / 32), kt = i % (KS * BN / 32) / (BN / 32), rg = i % (BN / 32);
    // Lane l carries k-half l / 32 of row l % 32, so each 32-row group lands
    // in LDS as [k-half][row][16 bytes] and a fragment read (16 lanes = 16
    // consecutive rows of one half) covers 256 contiguous bytes: no bank
    // conflicts ([row][half] order gave every pass a two-way conflict).
    const int row = rg * 32 + (lane & 31);
    b_voff[q] = n0 + row < p.N ? (int)((pl * KN + (long)kt * p.N * 16 + (long)(n0 + row) * 16 + 8 * (lane >> 5)) * 2)
                               : INT_MIN;
    b_lds[q] = pl * PLANE_B + kt * BN * 32 + rg * 1024;
  }
  auto issue = [&](int stage, int k0) {
    char* As = smem + stage * STAGE;
    char* Bs = As + STAGE_A;
    const int tap = k0 / p.C_in;  // uniform: a k-tile lies in one tap
    if (a_buf) {
      const int tap_off = tap * p.C_in * 4, soff = k0 * 4 - tap_off;
#pragma unroll
      for (int i = 0; i < AI; ++i) {
        const bool ok = (unsigned)(a_p0[i] + tap) < (unsigned)p.L_in;
        fm_buf_load_lds16(ra, As + (wave * AI + i) * RPI * BK * 4, ok ? a_voff[i] + tap_off : INT_MIN, soff);
      }
    } else {
#pragma unroll
      for (int i = 0; i < AI; ++i) {
        const bool ok = (unsigned)(a_p0[i] + tap) < (unsigned)p.L_in;
        const float* src = ok ? a_row[i] + k0 : g_zero16;
        __builtin_amdgcn_global_load_lds((__attribute__((address_space(1))) void*)src,
                                         (__attribute__((address_space(3))) void*)(As + (wave * AI + i) * RPI * BK * 4),
                                         16, 0, 0);
      }
    }
    // B: per-lane offsets fixed for the whole loop, the k-tile's place in
    // the planes as the scalar offset; past-N columns read out of range (zero).
    const int soff = (k0 >> 4) * p.N * 32;
#pragma unroll
    for (int q = 0; q < NBW; ++q) {
      const int i = wave + q * NW;
      if (i < NBI)
        fm_buf_load_lds16(rb, Bs + b_lds[q], b_voff[q], soff);
    }
  };

  floatx16 acc[FM][FN];
#pragma unroll
  for (int i = 0; i < FM; ++i)
#pragma unroll
    for (int j = 0; j < FN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int lrow = lane & 31, lk = lane >> 5;
  constexpr bool elu_in = ELU;  // ELU on load (a separate instantiation)
  const int nkt = (k_end - k_begin) / BK;
  if (nkt > 0) issue(0, k_begin);
  for (int kt = 0; kt < nkt; ++kt) {
    // This wave's loads of stage kt are done; after the barrier every wave's
    // are, and every wave has finished reading stage (kt + 1) % 2.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
    if (kt + 1 < nkt) issue((kt + 1) % NST, k_begin + (kt + 1) * BK);
    const char* As = smem + (kt % NST) * STAGE;
    const char* Bs = As + STAGE_A;
#pragma unroll
    for (int ks = 0; ks < KS; ++ks) {
      bf16x8 a0[FM], a1[FM], a2[FM], b0[FN], b1[FN], b2[FN];
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int row = wm0 + 32 * i + lrow;
        const int sw = (row / SWR) & (CPR - 1);
        floatx4 v0 = *reinterpret_cast<const floatx4*>(As + row * BK * 4 + 16 * ((4 * ks + 2 * lk) ^ sw));
        floatx4 v1 = *reinterpret_cast<const floatx4*>(As + row * BK * 4 + 16 * ((4 * ks + 2 * lk + 1) ^ sw));
        if (elu_in) {
#pragma unroll
          for (int e = 0; e < 4; ++e) v0[e] = fm_elu(v0[e]), v1[e] = fm_elu(v1[e]);
        }
        bf16x4 l0, l1, l2, h0, h1, h2;
        split3(v0, l0, l1, l2);
        split3(v1, h0, h1, h2);
        a0[i] = __builtin_shufflevector(l0, h0, 0, 1, 2, 3, 4, 5, 6, 7);
        a1[i] = __builtin_shufflevector(l1, h1, 0, 1, 2, 3, 4, 5, 6, 7);
        a2[i] = __builtin_shufflevector(l2, h2, 0, 1, 2, 3, 4, 5, 6, 7);
      }
#pragma unroll
      for (int j = 0; j < FN; ++j) {
        const char* bb = Bs + ks * BN * 32 + (wn0 + 32 * j) * 32 + lk * 512 + lrow * 16;
        b0[j] = *reinterpret_cast<const bf16x8*>(bb);
        b1[j] = *reinterpret_cast<const bf16x8*>(bb + PLANE_B);
        b2[j] = *reinterpret_cast<const bf16x8*>(bb + 2 * PLANE_B);
      }
      // Waves issuing their products run at raised priority, so a SIMD's
      // MFMA pipe is fed before another wave's split: in the 64- and 128-row
      // tiles (C3 128x128 ELU-on-load 172 -> 159 us, split 32-deep 128x128
      // 352 -> 333 us).  Not in the 192x128 tile (1-2% slower) nor the
      // 256x128 one (at its 128-VGPR budget the change made it spill in the
      // k-loop).
      constexpr bool PRIO = BM <= 128;
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          acc[i][j] = fm_mfma32_bf16(a1[i], b1[j], acc[i][j]);
          acc[i][j] = fm_mfma32_bf16(a1[i], b0[j], acc[i][j]);
          acc[i][j] = fm_mfma32_bf16(a0[i], b1[j], acc[i][j]);
        }
#pragma unroll
      for (int i = 0; i < FM; ++i)
#pragma unroll
        for (int j = 0; j < FN; ++j) {
          acc[i][j] = fm_mfma32_bf16(a2[i], b0[j], acc[i][j]);
          acc[i][j] = fm_mfma32_bf16(a0[i], b2[j], acc[i][j]);
          acc[i][j] = fm_mfma32_bf16(a0[i], b0[j], acc[i][j]);
        }
      if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
    }
  }
  // Epilogue straight from the accumulators (no LDS pass, no barrier): lane
  // l of a 32x32 accumulator holds column l % 32 of rows
  // 8 (r / 4) + 4 (l / 32) + r % 4, so each store instruction writes two
  // 128-byte row segments.  Stores and residual loads go through buffer
  // resources over this tile's rows, so past-M rows and past-N columns
  // (offset INT_MIN) are dropped / read as zero without a branch.  An
  // accumulator's residuals are all loaded before its first store, its RoPE
  // factors eight rows at a time: the compiler does not move a load above a
  // store to y (which may alias the residual), so each would otherwise wait
  // out a memory round trip.  RoPE's partner column c ^ 32 of a 64-column head is the same
  // lane's accumulator of the neighbouring 32-column tile (wave tiles start
  // on 64-column boundaries).
  const int lcol = lane & 31;
  float* part = p.partial ? p.partial + (long)blockIdx.y * M * p.N : nullptr;
  const bool has_res = (p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE)) && !part;
  const bool scaled = (p.flags & FM_EPI_RES_SCALE) && !part;
  const int tile_bytes = (int)min((long)BM, M - m0) * p.N * 4;
  const __amdgpu_buffer_rsrc_t ry = fm_buffer((part ? part : p.y) + m0 * p.N, tile_bytes);
  const __amdgpu_buffer_rsrc_t rr = fm_buffer(has_res ? p.res + m0 * p.N : p.y, has_res ? tile_bytes : 0);
  // Cropped outputs: row m = b rows + t goes to row b y_rows + t when
  // t < y_rows; over a tile those rows rise by at most one per row, so they
  // lie within BM + 1 rows of the tile's first one (crop0).
  int crop0 = 0;
  if (p.y_rows != p.rows) {
    const int b0 = (int)fm_div((unsigned)m0, p.rows_div);
    crop0 = b0 * p.y_rows + min((int)m0 - b0 * p.rows, p.y_rows);
  }
  const __amdgpu_buffer_rsrc_t rc = fm_buffer(p.y + (long)crop0 * p.N, (BM + 1) * p.N * 4);
  static_assert(WTN % 64 == 0, "RoPE partners within the wave tile");
  auto epilogue = [&](auto crop_c, auto rope_c) {
    constexpr bool CROP = decltype(crop_c)::value, ROPE = decltype(rope_c)::value;
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int c = wn0 + 32 * j + lcol;
      const int n = n0 + c;
      const bool n_ok = n < p.N;
      const int ncl = n_ok ? n : 0;
      const bool rope = ROPE && n < p.rope_cols;
      const float bias = (p.bias && !part) ? p.bias[ncl % p.bias_len] : 0.0f;
      const float scale = scaled ? p.scale[ncl] : 0.0f;
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int rb = wm0 + 32 * i;
        // Lane offset of the accumulator's first row; row 8 (r / 4) + r % 4
        // further down is a wave-uniform scalar offset.
        const int voff = n_ok ? ((rb + 4 * (lane >> 5)) * p.N + n) * 4 : INT_MIN;
        auto soff = [&](int r) { return (8 * (r >> 2) + (r & 3)) * p.N * 4; };
        float res[16];
#pragma unroll
        for (int r = 0; r < 16; ++r) res[r] = (!ROPE && has_res) ? fm_buf_load1(rr, voff, soff(r)) : 0.0f;
        // RoPE factors in two halves of eight rows (all sixteen at once
        // would spill).
        float cs[8], sn[8];
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = acc[i][j][r];
          if constexpr (ROPE) {
            if (r % 8 == 0) {
#pragma unroll
              for (int q = 0; q < 8; ++q) {
                const int m = (int)min(m0 + rb + fm_mfma32_row(r + q, lane), M - 1);
                const int t = m - (int)fm_div((unsigned)m, p.seq_div) * p.rows_per_seq;
                cs[q] = rope ? p.rope_cos[t * 64 + (c & 63)] : 1.0f;
                sn[q] = rope ? p.rope_sin[t * 64 + (c & 63)] : 0.0f;
              }
            }
            // x*cos - x[d+32]*sin for d < 32, x*cos + x[d-32]*sin after; each
            // product and the sum rounded separately.
            const float pv = acc[i][j ^ 1][r];
            if (rope) v = __fadd_rn(__fmul_rn(v, cs[r % 8]), __fmul_rn((j & 1) ? pv : -pv, sn[r % 8]));
          }
          if (!part) v = epilogue_v(v, bias, res[r], scale, p.flags);
          if constexpr (CROP) {
            const int m = (int)m0 + rb + fm_mfma32_row(r, lane);
            const int b = (int)fm_div((unsigned)m, p.rows_div);
            const int t = m - b * p.rows;
            const bool ok = m < M && n_ok && t < p.y_rows;
            fm_buf_store1(v, rc, ok ? ((b * p.y_rows + t - crop0) * p.N + n) * 4 : INT_MIN, 0);
          } else {
            fm_buf_store1(v, ry, voff, soff(r));
          }
        }
      }
    }
  };
  using yes = std::true_type;
  using no = std::false_type;
  const bool crop = p.y_rows != p.rows && !part;
  if (!ELU && (p.flags & FM_EPI_ROPE)) {
    if (crop) epilogue(yes{}, yes{});
    else epilogue(no{}, yes{});
  } else {
    if (crop) epilogue(yes{}, no{});
    else epilogue(no{}, no{});
  }
}

// ---------------------------------------------------------------------------
// Single-input-channel causal conv (the waveform -> num_filters first layer):
// y[b, t, c] = bias[c] + sum_j w[c, j] * x[b, t - pad + j].  HBM-bound on the
// output; a block stages its 256 positions plus the causal halo in LDS and
// writes 4 channels per thread with 16-byte stores.
template <int K>
__global__ __launch_bounds__(256) void conv_cin1_kernel(const float* __restrict__ x, int L,
                                                        const float* __restrict__ w,  // [C][K]
                                                        const float* __restrict__ bias, int C,
                                                        int flags, float* __restrict__ y) {
  constexpr int TB = 256;
  __shared__ float xs[TB + K];
  const long b = blockIdx.y;
  const int t0 = blockIdx.x * TB;
  const int groups = C / 4;           // threads per row; divides 256 (C in {4,8,...,1024})
  const int rows_per_pass = 256 / groups;
  const int c = (threadIdx.x % groups) * 4;
  const int r0 = threadIdx.x / groups;
  float wr[4][K], bv[4];
#pragma unroll
  for (int u = 0; u < 4; ++u) {
    bv[u] = bias ? bias[c + u] : 0.0f;
#pragma unroll
    for (int j = 0; j < K; ++j) wr[u][j] = w[(c + u) * K + j];
  }
  for (int i = threadIdx.x; i < TB + K - 1; i += 256) {
    const int t = t0 - (K - 1) + i;
    xs[i] = (t >= 0 && t < L) ? x[b * L + t] : 0.0f;
  }
  __syncthreads();
  for (int r = r0; r < TB; r += rows_per_pass) {
    const int t = t0 + r;
    if (t >= L) break;
    float acc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      acc[u] = bv[u];
#pragma unroll
      for (int j = 0; j < K; ++j) acc[u] = fmaf(wr[u][j], xs[r + j], acc[u]);
    }
    floatx4 v = {acc[0], acc[1], acc[2], acc[3]};
    if (flags & FM_EPI_ELU) v = floatx4{fm_elu(v.x), fm_elu(v.y), fm_elu(v.z), fm_elu(v.w)};
    *reinterpret_cast<floatx4*>(y + (b * L + t) * (long)C + c) = v;
  }
}

// Single-output-channel causal conv (the num_filters -> waveform last layer):
// y[b, t] = bias + sum_{j, c} w[j*C + c] * act(x[b, t - (K-1) + j, c]) for t < y_len.
// Each input row is read once: a block stages rows t0-(K-1) .. t0+OUT-1 with
// four threads per row (a quarter of the channels each, 16-byte loads), every
// thread forms its row's contribution to all K taps, the four quarters combine
// in order, and output t0+i sums tap j of row i+j over j through LDS.
template <int C, int K>
__global__ __launch_bounds__(256) void conv_cout1_kernel(const float* __restrict__ x, int L,
                                                         const float* __restrict__ w,
                                                         const float* __restrict__ bias,
                                                         int flags, int y_len,
                                                         float* __restrict__ y) {
  constexpr int CQ = C / 4;            // channels per thread
  constexpr int ROWS = 64;             // staged rows per block
  constexpr int OUT = ROWS - (K - 1);  // outputs per block
  __shared__ float D[ROWS][K];
  const long b = blockIdx.y;
  const int t0 = blockIdx.x * OUT;
  const int r = threadIdx.x / 4, part = threadIdx.x % 4;
  const int tin = t0 - (K - 1) + r;
  const bool ok = tin >= 0 && tin < L;
  const float* row = x + (b * L + (ok ? tin : 0)) * (long)C + part * CQ;
  floatx4 v[CQ / 4];
#pragma unroll
  for (int c = 0; c < CQ / 4; ++c)
    v[c] = ok ? *reinterpret_cast<const floatx4*>(row + 4 * c) : floatx4{0.0f, 0.0f, 0.0f, 0.0f};
  float wr[K][CQ];
#pragma unroll
  for (int j = 0; j < K; ++j)
#pragma unroll
    for (int c = 0; c < CQ; ++c) wr[j][c] = w[j * C + part * CQ + c];
  if (flags & FM_ELU_IN) {
#pragma unroll
    for (int c = 0; c < CQ / 4; ++c) v[c] = floatx4{fm_elu(v[c].x), fm_elu(v[c].y), fm_elu(v[c].z), fm_elu(v[c].w)};
  }
#pragma unroll
  for (int j = 0; j < K; ++j) {
    float acc = 0.0f;
#pragma unroll
    for (int c = 0; c < CQ / 4; ++c) {
      acc = fmaf(wr[j][4 * c], v[c].x, acc);
      acc = fmaf(wr[j][4 * c + 1], v[c].y, acc);
      acc = fmaf(wr[j][4 * c + 2], v[c].z, acc);
      acc = fmaf(wr[j][4 * c + 3], v[c].w, acc);
    }
    // Ordered combine of the four quarters.
    const float p1 = __shfl_down(acc, 1, 4), p2 = __shfl_down(acc, 2, 4), p3 = __shfl_down(acc, 3, 4);
    if (part == 0) D[r][j] = __fadd_rn(__fadd_rn(__fadd_rn(acc, p1), p2), p3);
  }
  __syncthreads();
  if (threadIdx.x < OUT) {
    const int i = threadIdx.x, t = t0 + i;
    if (t < y_len) {
      float s = D[i][0];
#pragma unroll
      for (int j = 1; j < K; ++j) s = __fadd_rn(s, D[i + j][j]);
      if (bias) s = __fadd_rn(s, bias[0]);
      y[b * y_len + t] = s;
    }
  }
}

struct TileCfg {
  int BM, BN, WK, BK, id;
  long fill;  // fewest tiles for which this candidate is taken
};
// Candidates, largest first: the first whose tile count reaches its `fill`
// wins.  The 256x64 tile (two 512-thread blocks per CU) measured faster than
// every other shape from ~190 tiles (not at 128 with long K), so it is taken
// from 160 tiles.
constexpr TileCfg kTiles[] = {{256, 64, 1, 32, 6, 160},  {128, 128, 1, 64, 0, 224},
                              {128, 64, 1, 64, 1, 224},  {128, 32, 1, 64, 2, 224},
                              {32, 64, 4, 32, 3, 0}};
constexpr TileCfg kSplitTile = kTiles[4];
constexpr TileCfg kBigTile = kTiles[0];
constexpr TileCfg kBigSquare = {128, 128, 1, 32, 9, 160};  // double-buffered, for N >= 128
constexpr TileCfg kMid64 = {64, 64, 1, 128, 7, 0};
constexpr TileCfg kMid32 = {32, 32, 4, 128, 8, 0};
constexpr TileCfg kBig192 = {192, 128, 1, 32, 10, 0};  // double-buffered, one block per CU
constexpr TileCfg kBig64 = {64, 128, 1, 32, 11, 0};    // double-buffered, 32x32 per wave
// Direct-load forms of the three double-buffered tiles (taken when the
// operands allow, see gemm_dl_kernel).
constexpr TileCfg kDl128 = {128, 128, 1, 32, 13, 0};
constexpr TileCfg kX6 = {128, 128, 1, 32, 16, 0};     // bf16x6 tiles (k-tile 16; splits stay 32-aligned); direct-load A
constexpr TileCfg kX6Big = {256, 128, 1, 32, 17, 0};
constexpr TileCfg kX6Small = {64, 128, 1, 32, 18, 0};  // direct-load A, four waves of 32x64
constexpr TileCfg kX6Wide = {192, 128, 1, 32, 19, 0};  // direct-load A, twelve waves, one block per CU
// kX6 / kX6Wide with 32-deep k-tiles (80 / 96 KB of LDS: still two / one
// block per CU).
constexpr TileCfg kX6K32 = {128, 128, 1, 32, 20, 0};
constexpr TileCfg kX6WideK32 = {192, 128, 1, 32, 22, 0};
constexpr TileCfg kDl192 = {192, 128, 1, 32, 14, 0};
// 64x128 runs one block per CU: 64-deep k-tiles (96 KB ring) halve its barriers.
constexpr TileCfg kDl64 = {64, 128, 1, 64, 15, 0};


long tile_count(long M, int N, const TileCfg& t) {
  return ((M + t.BM - 1) / t.BM) * ((N + t.BN - 1) / t.BN);
}

// Relative MFMA efficiency of a tile at full occupancy (measured on the
// transformer and SEANet shapes): the per-CU work model below divides by it.
double tile_eff(int id) {
  switch (id) {
    case 9: case 6: return 1.0;
    case 10: return 0.95;
    case 11: return 0.85;
    case 7: case 0: case 1: case 2: return 0.7;
    case 8: return 0.6;
    default: return 0.55;
  }
}

// Work of the busiest CU (tiles dealt over 256 CUs), in output elements per
// unit of efficiency; K is common to all candidates.
double cu_load(long M, int N, const TileCfg& t) {
  const long per_cu = (tile_count(M, N, t) + 255) / 256;
  return (double)per_cu * t.BM * t.BN / tile_eff(t.id);
}

// Smallest power-of-two K-split (<= cap) that brings tiles * splits to
// `blocks`, keeping at least `min_k` reduction elements per split.
int pick_splits(long tiles, int K, long blocks, int cap, int min_k) {
  int s = 1;
  while (s < cap && tiles * s < blocks && K / (2 * s) >= min_k) s *= 2;
  return s;
}

// The kernel the last run_gemm call on this host thread launched (for
// fm_gemm_last_plan): instantiation name, grid and K-split count.
thread_local char g_last_plan[160] = "";

const char* kernel_name(int id, bool elu) {
  switch (id) {
    case 0: return "gemm_fast_kernel<128,128,2,2,1,64>";
    case 1: return "gemm_fast_kernel<128,64,4,1,1,64>";
    case 2: return "gemm_fast_kernel<128,32,4,1,1,64>";
    case 3: return "gemm_fast_kernel<32,64,1,1,4,32>";
    case 6: return "gemm_big_kernel<256,64,4,2,false>";
    case 9: return "gemm_big_kernel<128,128,2,4,true>";
    case 10: return "gemm_big_kernel<192,128,2,4,true>";
    case 11: return "gemm_big_kernel<64,128,2,4,true>";
    case 13: return "gemm_dl_kernel<128,128,4,32,2,4>";
    case 14: return "gemm_dl_kernel<192,128,4,32,2,4>";
    case 15: return "gemm_dl_kernel<64,128,4,64,2,4>";
    case 16: return elu ? "gemm_x6d_kernel<128,128,4,1,2,true>" : "gemm_x6d_kernel<128,128,4,2,2,false>";
    case 17: return elu ? "gemm_x6d_kernel<256,128,8,1,2,true>" : "gemm_x6d_kernel<256,128,8,1,2,false>";
    case 18: return elu ? "gemm_x6d_kernel<64,128,2,2,2,true>" : "gemm_x6d_kernel<64,128,2,2,2,false>";
    case 19: return elu ? "gemm_x6d_kernel<192,128,6,2,2,true>" : "gemm_x6d_kernel<192,128,6,2,2,false>";
    case 20: return "gemm_x6d_kernel<128,128,4,2,2,false,2>";
    case 22: return "gemm_x6d_kernel<192,128,6,2,2,false,2>";
    case 7: return "gemm_mid_kernel<64,64,1>";
    case 8: return "gemm_mid_kernel<32,32,4>";
    default: return "gemm_generic_kernel";
  }
}

void record_plan(int id, bool elu, long tiles, int splits) {
  snprintf(g_last_plan, sizeof g_last_plan, "%s tiles=%ld splits=%d%s", kernel_name(id, elu), tiles,
           splits, splits > 1 ? " +split-K reduce" : "");
}

int run_gemm(GemmArgs p, float* workspace, size_t workspace_bytes, hipStream_t s) {
  if (!p.x || !p.w || !p.y || p.batch < 0 || p.rows < 0 || p.K <= 0 || p.N <= 0 ||
      p.C_in <= 0 || p.L_in < 0 || p.rs <= 0 || p.y_rows < 0 || p.y_rows > p.rows)
    return FM_BAD_ARGUMENT;
  if ((p.flags & (FM_EPI_RES_ADD | FM_EPI_RES_SCALE)) && !p.res) return FM_BAD_ARGUMENT;
  if ((p.flags & FM_EPI_RES_SCALE) && !p.scale) return FM_BAD_ARGUMENT;
  // RoPE rides only on plain projections (no ELU on load, no residual).
  if ((p.flags & FM_EPI_ROPE) && (p.flags & (FM_ELU_IN | FM_EPI_RES_ADD | FM_EPI_RES_SCALE)))
    return FM_UNSUPPORTED;
  if (p.bias && p.bias_len <= 0) return FM_BAD_ARGUMENT;
  const long M = (long)p.batch * p.rows;
  if (M == 0 || p.y_rows == 0) return FM_OK;
  if (p.L_in == 0 || M > INT_MAX / 2) return FM_BAD_ARGUMENT;

  p.rows_div = fm_divisor((unsigned)p.rows);
  p.seq_div = fm_divisor((unsigned)(p.rows_per_seq > 0 ? p.rows_per_seq : 1));
  const bool fast = (p.C_in % 4 == 0) && (p.K % 4 == 0);
  TileCfg cfg = kSplitTile;
  long tiles = 0;
  int splits = 1;
  const bool big_ok = p.N % 4 == 0 && !(p.bias && p.bias_len % 4);
  const TileCfg big = p.N >= 128 ? kBigSquare : kBigTile;
  const long big_tiles = tile_count(M, p.N, big);
  if (!fast) {
    cfg = TileCfg{64, 64, 1, 16, -1, 0};
    tiles = tile_count(M, p.N, cfg);
  } else if (p.K >= 1024 && big_tiles < 384 && M >= 1024 && big_ok && workspace) {
    // Long K, a few hundred rows-bands of work: 256x64 tiles split along K
    // to ~512 blocks (two per CU).
    cfg = big;
    tiles = big_tiles;
    splits = pick_splits(tiles, p.K, 512, 8, 128);
    // When the 64x128 tile gives every CU exactly one tile and K is at most
    // 2048, it runs unsplit: no partials and no reduce launch (the
    // transformer's fc2 at 4000 rows: 79 us against 73 + 10 us split).
    const long t64 = tile_count(M, p.N, kBig64);
    if (p.K <= 2048 && t64 >= 240 && t64 <= 256) {
      cfg = kBig64;
      tiles = t64;
      splits = 1;
    }
  } else if (p.K >= 1024 && M < 1024 && p.N >= 1024 && big_ok && workspace) {
    // Few rows, long K, wide output (the 12.5-25 Hz convs into 1024+
    // columns): the 128x128 tile split along K to ~256 blocks measured
    // 4-6 us faster than the 64x64 mid tile (enc.down8, dec.first, dec.up8).
    cfg = big;
    tiles = big_tiles;
    splits = pick_splits(tiles, p.K, 256, 16, 128);
  } else if (p.K >= 1024 && M < 1024 && workspace) {
    // Few rows, long K: 64x64 (or, up to 128 rows, 32x32 with the K split
    // inside the block) 16x16-MFMA tiles split along K to ~384 blocks.
    cfg = M <= 128 ? kMid32 : kMid64;
    tiles = tile_count(M, p.N, cfg);
    splits = pick_splits(tiles, p.K, 384, 16, 384);
  } else {
    // Largest tile that still fills the GPU; tiles more than 2x wider than
    // the output are skipped (the narrowest fallback is always eligible).
    for (const TileCfg& t0 : kTiles) {
      const TileCfg& t = t0.id == 6 ? big : t0;
      if (t.WK == 1 && t.BN > 32 && t.BN / 2 >= p.N) continue;
      // The large tiles' float4 epilogue needs 4-aligned rows and bias periods.
      if (t.id == 6 || t.id == 9) {
        if (!big_ok) continue;
      }
      cfg = t;
      tiles = tile_count(M, p.N, t);
      if (tiles >= t.fill) break;
    }
    // A 128-row fast tile with K of a few hundred loses to the 64x64
    // 16x16-MFMA tile once that one has a few hundred tiles (measured on the
    // transformer's output projection at 2500-4000 rows).
    if ((cfg.id == 0 || cfg.id == 1 || cfg.id == 2) && p.K >= 256 && tile_count(M, p.N, kMid64) >= 384) {
      cfg = kMid64;
      tiles = tile_count(M, p.N, cfg);
    }
    // Few-hundred-tile shapes: the tile whose busiest CU does the least work
    // (a 192x128 tile gives the 4000-row qkv projection one tile per CU; 64x128
    // spreads the 512-column output projection over all CUs).  Switches only
    // on a clear (10%) predicted gain.
    if (big_ok && M >= 1024) {
      double best = cu_load(M, p.N, cfg);
      for (const TileCfg& t : {kBigSquare, kBig192, kBig64}) {
        const double l = cu_load(M, p.N, t);
        if (l < 0.9 * best) {
          best = l;
          cfg = t;
        }
      }
      tiles = tile_count(M, p.N, cfg);
    }
    // Global K-split for long K when even the K-split tile leaves CUs idle.
    const int kchunks = (p.K + KT - 1) / KT;
    if (cfg.WK > 1 && tiles < 384 && kchunks >= 32 && workspace)
      splits = (int)std::min<long>((512 + tiles - 1) / tiles, kchunks / 16);
  }
  // The direct-load tiles need every k-tile (32 deep) inside one tap.
  const bool dl_ok = big_ok && !(p.flags & (FM_REPLICATE | FM_ELU_IN)) && p.C_in % 32 == 0 &&
                     p.K % 32 == 0;
  if (dl_ok) {
    if (cfg.id == 9) cfg = kDl128;
    if (cfg.id == 10) cfg = kDl192;
    if (cfg.id == 11 && p.C_in % 64 == 0 && p.K % 64 == 0) cfg = kDl64;
    // With split weights the direct-load tiles become the bf16x6 tile.
  }
  // With split weights the large tiles become bf16x6 tiles (which also take
  // ELU on load: the A operand passes through registers) when that still
  // gives most CUs a tile (K-split blocks included); the few-hundred-tile
  // shapes keep the FP32 tile
  // picked for them (measured: the 512-column projections at 2500-4000 rows,
  // 64x128 FP32 tiles on all CUs against 80-128 bf16x6 tiles).
  // (The bf16x6 tiles address the weight planes through a buffer resource,
  // at most 2 GiB of planes, and store a tile's rows through 32-bit offsets:
  // 257 rows of N columns below 2 GiB.)
  const bool x6_ok = (p.flags & FM_WEIGHTS_X6) && big_ok && !(p.flags & FM_REPLICATE) &&
                     p.C_in % 16 == 0 && p.K % 16 == 0 && 6L * p.K * p.N <= 0x7fffffffL &&
                     257L * p.N * 4 <= 0x7fffffffL;
  if (x6_ok && cfg.id >= 9 && cfg.id <= 15 && cfg.id != 12) {
    const long t128 = tile_count(M, p.N, kX6);
    if (p.K >= 1024 && M >= 1024 && t128 < 360 && workspace) {
      // Long K over a few hundred tiles (the 2048-deep fc2 projection at
      // 2500-8000 rows, the 12-25 Hz convs): the bf16x6 tile split along K
      // to >= 360 blocks, 128x128 with at most 4 splits, else 64x128 with
      // at most 8 (>= 128 k per split).  Measured against the FP32 pick:
      // fc2 at 4000 rows 65 vs 77 us, at 2500 rows 50 vs 59 us; dec.up6 at
      // C2 61 vs 65 us.
      auto fewest = [&](const TileCfg& t, int most) {
        const long tc = tile_count(M, p.N, t);
        int sp = 1;
        while (sp < most && tc * sp < 360 && p.K / (2 * sp) >= 128) sp *= 2;
        return sp;
      };
      // From 160 tiles the direct-load 128x128 tile runs unsplit (no
      // partials, no reduce launch): C2 enc.down5 64 us against 70 us split,
      // C2 dec.up6 53 against 63 us, fc2 at 8000 rows 108 against 117 us.
      // At most one tile per CU with K >= 2048 splits in two instead, so
      // each CU holds two blocks (C3 enc.down8 495 -> 460 us, C4 dec.first
      // 178 -> 150 us).
      const int s128 = t128 < 160 ? fewest(kX6, 4) : (t128 <= 256 && p.K >= 2048) ? 2 : 1;
      if (t128 * s128 >= 360 || s128 == 1) {
        cfg = kX6;
        splits = s128;
        // Unsplit with two tiles on some CUs: 192x128 tiles, one per CU,
        // when they fit in one round, but not with ELU on load (there the
        // four-wave 128x128 tile at three blocks per CU wins: C4 res512.c1
        // at 20000 rows 124 against 130 us); unsplit with at most one tile
        // per CU: 64x128 tiles, so every CU works (C2 enc.down5 65 -> 57 us,
        // C2 dec.up6 52 -> 47 us).
        if (s128 == 1 && t128 > 256 && tile_count(M, p.N, kX6Wide) <= 256 && !(p.flags & FM_ELU_IN))
          cfg = kX6Wide;
        if (s128 == 1 && t128 <= 256) cfg = kX6Small;
      } else {
        cfg = kX6Small;
        splits = fewest(kX6Small, 8);
      }
      tiles = tile_count(M, p.N, cfg);
    } else if (t128 * splits >= 192) {
      // 256x128 where it gives >= 384 tiles, else the direct-load 128x128
      // tile (the 8000-row output projection 34 against 37 us for 64x128
      // tiles), or 192x128 (one per CU) where 128x128 would put two on some
      // CUs and 192x128 tiles fit in one round (4000-row qkv 54 -> 45 us), or
      // 64x128 where unsplit 128x128 tiles would leave CUs idle (2500-row qkv
      // 32-33 -> 29.6 us, C1 enc.down4 33.5-35 -> 30.7 us, C1 dec.up5
      // 33-34 -> 30.5 us).  Every bf16x6 tile accumulates an output element
      // in the same order, so the choice never changes a result.
      cfg = tile_count(M, p.N, kX6Big) >= 384 ? kX6Big : kX6;
      if (cfg.id == kX6.id && t128 > 256 && tile_count(M, p.N, kX6Wide) <= 256) cfg = kX6Wide;
      if (cfg.id == kX6.id && t128 <= 256 && splits == 1) cfg = kX6Small;
      tiles = tile_count(M, p.N, cfg);
    }
  }
  // The RoPE epilogue needs whole unsplit bf16x6 tiles (the partner columns
  // of a head sit in the neighbouring accumulator of the same wave).  Any other plan stays
  // as selected, so the projection rounds as fm_linear's, and RoPE follows
  // as its own launch.
  // 32-deep k-tiles (two 16-deep sub-tiles per stage, in k order, so the
  // result is the 16-deep tile's bit for bit) halve the barriers of the
  // 128x128 and 192x128 tiles at the same blocks per CU: C2 dec.up5 51.6 ->
  // 50.2 us, C3 enc.down8 368 -> 353 us, 4000-row qkv 40.9 -> 40.0 us,
  // 2500-row fc1 42.9 -> 41.4 us.  The 64x128 tile keeps 16 (its 64 KB ring
  // would cost blocks per CU: 2500-row fc2 46 -> 50 us).
  if (!(p.flags & FM_ELU_IN) && p.C_in % 32 == 0 && p.K % 32 == 0) {
    if (cfg.id == kX6.id) cfg = kX6K32;
    else if (cfg.id == kX6Wide.id) cfg = kX6WideK32;
  }
  const bool rope_after = (p.flags & FM_EPI_ROPE) && (!(cfg.id >= 16 && cfg.id <= 22) || splits != 1);
  if (rope_after) p.flags &= ~FM_EPI_ROPE;
  if (splits > 1) {
    const size_t per = (size_t)M * p.N * sizeof(float);
    while (splits > 1 && per * splits > workspace_bytes) --splits;
    splits = std::max(splits, 1);
  }
  // Split boundaries are multiples of the kernel's k-tile.
  const int kt = std::max(cfg.BK, KT);
  const int ktiles = (p.K + kt - 1) / kt;
  p.k_split = ((ktiles + splits - 1) / splits) * kt;
  splits = (p.K + p.k_split - 1) / p.k_split;
  p.partial = splits > 1 ? workspace : nullptr;

  dim3 grid((unsigned)tiles, splits);
  record_plan(cfg.id, (p.flags & FM_ELU_IN) != 0, tiles, splits);
  // Zero-page loader of the large tiles (their k-tile is 32).
  const bool zp = !(p.flags & FM_REPLICATE) && p.C_in % 32 == 0;
  switch (cfg.id) {
    case 0: hipLaunchKernelGGL((gemm_fast_kernel<128, 128, 2, 2, 1, 64>), grid, dim3(NTHREADS), 0, s, p); break;
    case 1: hipLaunchKernelGGL((gemm_fast_kernel<128, 64, 4, 1, 1, 64>), grid, dim3(NTHREADS), 0, s, p); break;
    case 2: hipLaunchKernelGGL((gemm_fast_kernel<128, 32, 4, 1, 1, 64>), grid, dim3(NTHREADS), 0, s, p); break;
    case 3: hipLaunchKernelGGL((gemm_fast_kernel<32, 64, 1, 1, 4, 32>), grid, dim3(NTHREADS), 0, s, p); break;
#define FM_BIG(BM_, BN_, WM_, WN_, DB_)                                                              \
  if (zp) hipLaunchKernelGGL((gemm_big_kernel<BM_, BN_, WM_, WN_, DB_, true>), grid, dim3(512), 0, s, p); \
  else hipLaunchKernelGGL((gemm_big_kernel<BM_, BN_, WM_, WN_, DB_, false>), grid, dim3(512), 0, s, p)
    case 6: FM_BIG(256, 64, 4, 2, false); break;
    case 9: FM_BIG(128, 128, 2, 4, true); break;
    case 10: FM_BIG(192, 128, 2, 4, true); break;
    case 11: FM_BIG(64, 128, 2, 4, true); break;
#undef FM_BIG
    case 13: hipLaunchKernelGGL((gemm_dl_kernel<128, 128, 4, 32, 2, 4>), grid, dim3(512), 0, s, p); break;
    case 14: hipLaunchKernelGGL((gemm_dl_kernel<192, 128, 4, 32, 2, 4>), grid, dim3(512), 0, s, p); break;
    case 15: hipLaunchKernelGGL((gemm_dl_kernel<64, 128, 4, 64, 2, 4>), grid, dim3(512), 0, s, p); break;
    case 16:
      // ELU on load: four waves of 32 x 128, so each A element's ELU and
      // split run once (C3 res512.c1 230 -> 191 us against two 32 x 64 waves).
      if (p.flags & FM_ELU_IN)
        hipLaunchKernelGGL((gemm_x6d_kernel<128, 128, 4, 1, 2, true>), grid, dim3(256), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      else
        hipLaunchKernelGGL((gemm_x6d_kernel<128, 128, 4, 2, 2, false>), grid, dim3(512), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      break;
    case 17:
      if (p.flags & FM_ELU_IN)
        hipLaunchKernelGGL((gemm_x6d_kernel<256, 128, 8, 1, 2, true>), grid, dim3(512), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      else
        hipLaunchKernelGGL((gemm_x6d_kernel<256, 128, 8, 1, 2, false>), grid, dim3(512), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      break;
    case 18:
      if (p.flags & FM_ELU_IN)
        hipLaunchKernelGGL((gemm_x6d_kernel<64, 128, 2, 2, 2, true>), grid, dim3(256), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      else
        hipLaunchKernelGGL((gemm_x6d_kernel<64, 128, 2, 2, 2, false>), grid, dim3(256), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      break;
    case 19:
      if (p.flags & FM_ELU_IN)
        hipLaunchKernelGGL((gemm_x6d_kernel<192, 128, 6, 2, 2, true>), grid, dim3(768), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      else
        hipLaunchKernelGGL((gemm_x6d_kernel<192, 128, 6, 2, 2, false>), grid, dim3(768), 0, s, p,
                           reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      break;
    case 20:
      hipLaunchKernelGGL((gemm_x6d_kernel<128, 128, 4, 2, 2, false, 2>), grid, dim3(512), 0, s, p,
                         reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      break;
    case 22:
      hipLaunchKernelGGL((gemm_x6d_kernel<192, 128, 6, 2, 2, false, 2>), grid, dim3(768), 0, s, p,
                         reinterpret_cast<const __bf16*>(p.w + (long)p.N * p.K));
      break;
    case 7: hipLaunchKernelGGL((gemm_mid_kernel<64, 64, 1>), grid, dim3(NTHREADS), 0, s, p); break;
    case 8: hipLaunchKernelGGL((gemm_mid_kernel<32, 32, 4>), grid, dim3(NTHREADS), 0, s, p); break;
    default: hipLaunchKernelGGL(gemm_generic_kernel, grid, dim3(256), 0, s, p); break;
  }
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return (int)e;
  if (splits > 1) {
    const long total = M * p.N;
    if (p.N % 4 == 0 && !(p.bias && p.bias_len % 4) && total / 4 < 0x7fffffffL) {
      const int blocks = (int)std::min<long>((total / 4 + 255) / 256, 2048);
      hipLaunchKernelGGL(splitk_reduce4_kernel, dim3(blocks), dim3(256), 0, s, p, splits,
                         fm_divisor((unsigned)(p.N / 4)));
    } else {
      const int blocks = (int)std::min<long>((total + 255) / 256, 2048);
      hipLaunchKernelGGL(splitk_reduce_kernel, dim3(blocks), dim3(256), 0, s, p, splits);
    }
    e = hipGetLastError();
    if (e != hipSuccess) return (int)e;
  }
  if (rope_after)
    return fm_apply_rope(p.y, M, p.N, p.rope_cols, 64, p.rope_cos, p.rope_sin, p.rows_per_seq, s);
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
  const int plain = p.flags & ~(FM_EPI_ELU | FM_ELU_IN | FM_WEIGHTS_X6);
  if (x && weight_packed && y && batch > 0 && length > 0 && stride == 1 && plain == 0 &&
      y_length >= 0 && y_length <= length) {
    // The packed layout W^T[c_out][(tap, c_in)] doubles as [C][k] / [k*C] here.
    if (in_channels == 1 && kernel == 7 && out_channels % 4 == 0 && out_channels <= 1024 &&
        256 % (out_channels / 4) == 0 && !(p.flags & FM_ELU_IN) && y_length == length) {
      hipLaunchKernelGGL(conv_cin1_kernel<7>, dim3((length + 255) / 256, batch), dim3(256), 0,
                         stream, x, length, weight_packed, bias, out_channels, p.flags, y);
      return (int)hipGetLastError();
    }
    if (out_channels == 1 && in_channels == 64 && kernel == 3 && !(p.flags & FM_EPI_ELU)) {
      if (y_length == 0) return FM_OK;
      hipLaunchKernelGGL((conv_cout1_kernel<64, 3>), dim3((y_length + 61) / 62, batch), dim3(256), 0,
                         stream, x, length, weight_packed, bias, p.flags, y_length, y);
      return (int)hipGetLastError();
    }
  }
  return run_gemm(p, workspace, workspace_bytes, stream);
}

// Conv1d over exactly the given rows (no implicit padding): output row t
// reads input rows t*stride .. t*stride + kernel - 1; output length
// (length - kernel) / stride + 1 per batch item.  Streaming convolution,
// where the caller prepends the layer's cached left context.
int fm_conv1d_valid(const float* x, int batch, int length, int in_channels,
                    const float* weight_packed, const float* bias, int out_channels, int kernel,
                    int stride, int flags, const float* residual, float* y, float* workspace,
                    size_t workspace_bytes, hipStream_t stream) {
  if (kernel <= 0 || stride <= 0 || length < kernel || (flags & (FM_REPLICATE | FM_EPI_RES_SCALE)))
    return FM_BAD_ARGUMENT;
  GemmArgs p{};
  p.x = x; p.w = weight_packed; p.bias = bias; p.res = residual; p.scale = nullptr; p.y = y;
  p.batch = batch; p.L_in = length; p.C_in = in_channels;
  p.rows = (length - kernel) / stride + 1;
  p.rs = stride; p.padL = 0; p.K = kernel * in_channels; p.N = out_channels;
  p.y_rows = p.rows; p.bias_len = out_channels; p.flags = flags;
  return run_gemm(p, workspace, workspace_bytes, stream);
}

// The bf16x6 planes of a packed weight W^T [rows][cols] (cols % 16 == 0):
// [3][cols/16][rows][16] bf16.  Callers store them right after the FP32
// weight and pass FM_WEIGHTS_X6 in flags.
int fm_gemm_last_plan(char* buf, int size) {
  if (!buf || size <= 0) return FM_BAD_ARGUMENT;
  snprintf(buf, (size_t)size, "%s", g_last_plan);
  return FM_OK;
}

int fm_split_weights(const float* weight_packed, int rows, int cols, void* planes, hipStream_t stream) {
  if (!weight_packed || !planes || rows <= 0 || cols <= 0) return FM_BAD_ARGUMENT;
  if (cols % 16) return FM_UNSUPPORTED;
  const long n4 = (long)rows * cols / 4;
  hipLaunchKernelGGL(split_weights_kernel, dim3((unsigned)((n4 + 255) / 256)), dim3(256), 0, stream,
                     weight_packed, rows, cols, reinterpret_cast<bf16x4*>(planes));
  return (int)hipGetLastError();
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
  p.flags = flags & ~(FM_REPLICATE | FM_ELU_IN | FM_EPI_ROPE);
  return run_gemm(p, workspace, workspace_bytes, stream);
}

int fm_linear_rope(const float* x, int rows, int in_features, const float* weight_packed,
                   int out_features, int flags, const float* cos_table, const float* sin_table,
                   int rope_cols, int rows_per_seq, float* y, float* workspace, size_t workspace_bytes,
                   hipStream_t stream) {
  if (!cos_table || !sin_table || rope_cols <= 0 || rope_cols % 64 || rope_cols > out_features ||
      out_features % 64 || rows_per_seq <= 0)
    return FM_BAD_ARGUMENT;
  if (flags != FM_WEIGHTS_X6) return FM_UNSUPPORTED;  // bf16x6 tiles only, no other epilogue
  GemmArgs p{};
  p.x = x; p.w = weight_packed; p.bias = nullptr; p.res = nullptr; p.scale = nullptr; p.y = y;
  p.batch = 1; p.L_in = rows; p.C_in = in_features; p.rows = rows; p.rs = 1; p.padL = 0;
  p.K = in_features; p.N = out_features; p.y_rows = rows; p.bias_len = 0;
  p.flags = FM_WEIGHTS_X6 | FM_EPI_ROPE;
  p.rope_cos = cos_table; p.rope_sin = sin_table; p.rope_cols = rope_cols; p.rows_per_seq = rows_per_seq;
  return run_gemm(p, workspace, workspace_bytes, stream);
}

}  // extern "C"
