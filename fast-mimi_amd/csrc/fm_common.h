// Shared device helpers for the gfx950 (CDNA4) Mimi kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>
#include <climits>
#include <algorithm>
#include <mutex>

#define FM_DEVICE __device__ __forceinline__

typedef float floatx4 __attribute__((ext_vector_type(4)));
typedef float floatx16 __attribute__((ext_vector_type(16)));

// Status codes returned through the C ABI (hipError_t values pass through).
enum FmStatus {
  FM_OK = 0,
  FM_BAD_ARGUMENT = 1000,
  FM_WORKSPACE_TOO_SMALL = 1001,
  FM_UNSUPPORTED = 1002,
  FM_SCRATCH_LIMIT = 1003,  // input larger than an allocation-free entry point's fixed scratch
};

// Epilogue / loader flags of the implicit-GEMM kernel.
enum FmGemmFlags {
  FM_ELU_IN = 1,        // apply ELU to A operands as they are loaded
  FM_REPLICATE = 2,     // out-of-range input positions clamp to the edge (else zero)
  FM_EPI_ELU = 4,       // ELU on the output
  FM_EPI_GELU = 8,      // exact-erf GELU on the output
  FM_EPI_RES_ADD = 16,  // y = res + (acc + bias)
  FM_EPI_RES_SCALE = 32, // y = res + scale[n] * acc
  FM_WEIGHTS_X6 = 64,    // weight_packed is followed by its three bf16 planes (fm_split_weights)
  FM_ACT_EXP = 128,      // residual blocks: ELUs as e^x - 1 (fm_elu_exp), for decoder-side calls
  FM_EPI_ROPE = 256      // internal (fm_linear_rope): RoPE on the first rope_cols output columns
};

// e^x - 1 for x <= 0, branch-free.  Near zero (x > -1/4) x * q(x), q a
// degree-4 polynomial fitted to expm1(x) / x on [-1/4, 0] (iteratively
// reweighted least squares toward equal relative error; evaluated in FP32
// Horner form with FMAs it stays within 1.12 ulp of float64 expm1 over 4M
// samples of the interval, against 1.06 ulp for the degree-8 Taylor series);
// further out e^x - 1 from the hardware exponential, where the result is at
// least 0.22 in magnitude so the subtraction loses nothing.  Within a few ulp
// of expm1 over x <= 0.
FM_DEVICE float fm_expm1_neg(float x) {
  float p = fmaf(x, 0.007509505841881037f, 0.04148859530687332f);
  p = fmaf(x, p, 0.16665075719356537f);
  p = fmaf(x, p, 0.4999994933605194f);
  p = fmaf(x, p, 1.0f);
  const float small = x * p;
  const float large = __expf(x) - 1.0f;
  return x > -0.25f ? small : large;
}

// ELU with alpha = 1 (torch.nn.ELU): x for x > 0, e^x - 1 otherwise.  The
// expm1 branch is evaluated for every lane and selected (x > 0 only discards
// it; NaN propagates through it): a per-element branch would be taken by
// almost every wave anyway.
FM_DEVICE float fm_elu(float x) {
  const float r = fm_expm1_neg(x);
  return x > 0.0f ? x : r;
}

// ELU from the hardware exponential alone, e^x - 1 for x <= 0: an absolute
// error of a few 2^-24 near zero (where fm_elu keeps a relative one), for
// kernels held to an absolute bar rather than to bit-exact codes (the
// decoder's waveform).  Five instructions against fm_elu's twelve.
FM_DEVICE float fm_elu_exp(float x) {
  const float r = __expf(x) - 1.0f;
  return x > 0.0f ? x : r;
}

// Exact-erf GELU (torch.nn.functional.gelu, approximate='none').
FM_DEVICE float fm_gelu(float x) {
  return __fmul_rn(__fmul_rn(x, 0.5f), __fadd_rn(1.0f, erff(__fmul_rn(x, 0.70710678118654752440f))));
}

// One v_mfma_f32_32x32x2f32: D(32x32) += A(32x2) * B(2x32).
// Lane l supplies A[l % 32][l / 32] and B[l / 32][l % 32]; the 16 results of
// lane l are D[8*(r/4) + 4*(l/32) + (r%4)][l % 32], r = 0..15.
FM_DEVICE floatx16 fm_mfma32(float a, float b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x2f32(a, b, c, 0, 0, 0);
}

FM_DEVICE int fm_mfma32_row(int r, int lane) { return 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3); }

// bf16x6 primitives: one v_mfma_f32_32x32x16_bf16 (lane l supplies row / column
// l % 32, k = 8 (l / 32) .. +7, same result layout as fm_mfma32) and the
// three-piece round-to-nearest bf16 split of an FP32 value.
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));

FM_DEVICE floatx16 fm_mfma32_bf16(bf16x8 a, bf16x8 b, floatx16 c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c, 0, 0, 0);
}

// v = h0 + h1 + h2 (+ a residual below 2^-24 |v|), each a round-to-nearest bf16.
// Pairs are converted with one packed conversion whose two halves, widened
// back by a shift and a mask, give the residuals: the same values as
// converting each element and widening it, in fewer instructions.
FM_DEVICE void split3(floatx4 v, bf16x4& h0, bf16x4& h1, bf16x4& h2) {
  typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
  typedef float floatx2_t __attribute__((ext_vector_type(2)));
  typedef unsigned uintx2_t __attribute__((ext_vector_type(2)));
  auto pack = [](float a, float b) {
    return __builtin_bit_cast(unsigned, __builtin_convertvector((floatx2_t{a, b}), bf16x2_t));
  };
  auto lo = [](unsigned u) { return __builtin_bit_cast(float, u << 16); };
  auto hi = [](unsigned u) { return __builtin_bit_cast(float, u & 0xffff0000u); };
  unsigned p0[2], p1[2], p2[2];
#pragma unroll
  for (int q = 0; q < 2; ++q) {
    const float a = v[2 * q], b = v[2 * q + 1];
    p0[q] = pack(a, b);
    const float ra = a - lo(p0[q]), rb = b - hi(p0[q]);
    p1[q] = pack(ra, rb);
    p2[q] = pack(ra - lo(p1[q]), rb - hi(p1[q]));
  }
  h0 = __builtin_bit_cast(bf16x4, (uintx2_t{p0[0], p0[1]}));
  h1 = __builtin_bit_cast(bf16x4, (uintx2_t{p1[0], p1[1]}));
  h2 = __builtin_bit_cast(bf16x4, (uintx2_t{p2[0], p2[1]}));
}

static inline int fm_ceil_div(long a, long b) { return (int)((a + b - 1) / b); }

// Division by a runtime constant d >= 1 for numerators n < 2^31:
// n / d = (umulhi(magic, n) + n) >> shift with shift = ceil(log2 d) and
// magic = floor(2^32 (2^shift - d) / d) + 1 (the round-up method of Granlund
// and Montgomery; t + n stays below 2^32 because t <= n < 2^31).  Three vector
// instructions instead of a ~30-instruction integer division.
struct FmDivisor {
  unsigned magic;
  int shift;
};
static inline FmDivisor fm_divisor(unsigned d) {
  int l = 0;
  while ((1ull << l) < d) ++l;
  const unsigned long long m = ((1ull << 32) * ((1ull << l) - d)) / d + 1;
  return FmDivisor{(unsigned)m, l};
}
FM_DEVICE unsigned fm_div(unsigned n, FmDivisor d) {
  return (__umulhi(d.magic, n) + n) >> d.shift;
}

// Raw buffer (gfx9 descriptor word 3 = 0x00020000) over `bytes` bytes at
// `base`.  An access is a per-lane 32-bit byte offset plus a wave-uniform one
// (an SGPR: compile-time row offsets cost no vector instructions).  Callers
// keep every access inside the buffer.
FM_DEVICE __amdgpu_buffer_rsrc_t fm_buffer(const void* base, int bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}
FM_DEVICE floatx4 fm_buf_load4(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(floatx4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}
// 16 bytes per lane from a buffer straight into LDS (lane l's bytes at
// lds + 16 l); out-of-range offsets read zeros.
FM_DEVICE void fm_buf_load_lds16(__amdgpu_buffer_rsrc_t r, void* lds, int voff, int soff) {
  __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (__attribute__((address_space(3))) void*)lds, 16, voff, soff, 0, 0);
}
FM_DEVICE float fm_buf_load1(__amdgpu_buffer_rsrc_t r, int voff, int soff) {
  return __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(r, voff, soff, 0));
}
FM_DEVICE void fm_buf_store1(float v, __amdgpu_buffer_rsrc_t r, int voff, int soff) {
  __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(unsigned, v), r, voff, soff, 0);
}

// Block barrier for LDS traffic only: this wave's LDS operations complete,
// then s_barrier.  Unlike __syncthreads it does not wait for the wave's
// outstanding global loads and stores (prefetches keep flying).
FM_DEVICE void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Orders this wave's LDS accesses: everything before completes before
// anything after is issued (the compiler may not move memory ops across).
FM_DEVICE void wave_lds_fence() {
  asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  __builtin_amdgcn_wave_barrier();
}

// ---------------------------------------------------------------------------
// Cross-block exchange inside one launch (persistent kernels).  Data that
// another block reads is stored and loaded as agent-scope relaxed atomics:
// the stores write through the caches to memory and the loads bypass them
// (the sc bits the compiler sets for that scope), so the exchange is coherent
// whichever XCD each block runs on, with no L2 write-back or invalidate, and
// the compiler still overlaps independent loads.  Arrivals are atomic adds on
// a counter; a waiter polls it with coherent loads, at most `spin` times.
FM_DEVICE void fm_store64_coherent(unsigned long long* p, unsigned long long v) {
  __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
FM_DEVICE unsigned long long fm_load64_coherent(const unsigned long long* p) {
  return __hip_atomic_load(const_cast<unsigned long long*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
// Called by one lane of the wave that issued the block's coherent stores:
// waits for them to complete, arrives, then polls until `target` arrivals
// (false on timeout).
FM_DEVICE bool fm_arrive_and_wait(unsigned* counter, unsigned target, long spin) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  for (long s = 0; s < spin; ++s)
    if (__hip_atomic_load(counter, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= target) return true;
  return false;
}
