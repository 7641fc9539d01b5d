// Host-side argument validation of the C ABI (include/fast_mimi_amd.h),
// built for the CPU under AddressSanitizer + UndefinedBehaviorSanitizer by
// tests/test_sanitize.py.  Every call below must be rejected (or be a no-op)
// before any HIP call is made, so no GPU is needed; the sanitizers check that
// the checks themselves read nothing out of bounds and that the size queries
// do not overflow.  Pointers that are never dereferenced are fake addresses.
#include <cstdint>
#include <cstdio>
#include <climits>

#include "fast_mimi_amd.h"

namespace {

int failures = 0;

void expect(const char* what, long got, long want) {
  if (got != want) {
    std::printf("FAIL %s: got %ld, want %ld\n", what, got, want);
    ++failures;
  }
}

}  // namespace

int main() {
  float* const P = reinterpret_cast<float*>(0x1000);  // never dereferenced
  int64_t* const C = reinterpret_cast<int64_t*>(0x2000);
  const hipStream_t S = nullptr;
  constexpr int BAD = 1000, WS = 1001, UNSUP = 1002, SCRATCH = 1003;

  // Convolutions.
  {
    char plan[8];
    expect("gemm_last_plan null buffer", fm_gemm_last_plan(nullptr, 8), BAD);
    expect("gemm_last_plan zero size", fm_gemm_last_plan(plan, 0), BAD);
    expect("gemm_last_plan small buffer", fm_gemm_last_plan(plan, (int)sizeof plan), 0);
  }
  expect("conv1d null x", fm_conv1d(nullptr, 1, 16, 64, P, nullptr, 64, 3, 1, 0, 0, nullptr, P, 16, P, 1 << 20, S), BAD);
  expect("conv1d negative length", fm_conv1d(P, 1, -1, 64, P, nullptr, 64, 3, 1, 0, 0, nullptr, P, 16, P, 1 << 20, S), BAD);
  expect("conv1d empty batch", fm_conv1d(P, 0, 16, 64, P, nullptr, 64, 3, 1, 0, 0, nullptr, P, 16, P, 1 << 20, S), 0);
  expect("conv1d residual flag without residual",
         fm_conv1d(P, 1, 16, 64, P, nullptr, 64, 3, 1, 0, 16, nullptr, P, 16, P, 1 << 20, S), BAD);
  expect("conv_transpose1d kernel not a stride multiple",
         fm_conv_transpose1d(P, 1, 16, 64, P, nullptr, 32, 7, 2, 0, nullptr, P, P, 1 << 20, S), UNSUP);
  expect("conv1d_valid null y", fm_conv1d_valid(P, 1, 16, 64, P, nullptr, 64, 3, 1, 0, nullptr, nullptr, P, 1 << 20, S), BAD);
  expect("linear null weight", fm_linear(P, 4, 512, nullptr, 512, 0, nullptr, nullptr, P, P, 1 << 20, S), BAD);

  // Residual blocks.
  expect("resblock unsupported width", fm_resblock(P, 1, 16, 96, P, P, P, P, 1, P + 64, S), UNSUP);
  expect("resblock in place", fm_resblock(P, 1, 16, 128, P, P, P, P, 1, P, S), BAD);
  expect("resblock64_conv small workspace",
         fm_resblock64_conv(P, 1, 4096, P, P, P, P, 1, P, nullptr, 4096, P, P, 8, S), WS);
  expect("conv_resblock64 empty", fm_conv_resblock64(P, 0, 4096, P, P, P, P, P, P, 1, P, S), 0);

  // Transformer pieces.
  expect("row_linear unsupported width",
         fm_row_linear(P, 250, 300, nullptr, nullptr, 1e-5f, P, 512, 0, nullptr, nullptr, nullptr, nullptr, 0, 250, P, S), UNSUP);
  expect("row_linear gamma without beta",
         fm_row_linear(P, 250, 512, P, nullptr, 1e-5f, P, 512, 0, nullptr, nullptr, nullptr, nullptr, 0, 250, P, S), BAD);
  expect("row_linear_packed rope cols not whole heads",
         fm_row_linear_packed(P, 250, 512, nullptr, nullptr, 1e-5f, P, 1536, 0, nullptr, nullptr, P, P, 96, 250, P, S), BAD);
  expect("row_linear_packed LayerNorm at K 2048",
         fm_row_linear_packed(P, 250, 2048, P, P, 1e-5f, P, 512, 0, nullptr, nullptr, nullptr, nullptr, 0, 250, P, S), UNSUP);
  expect("row_linear_packed too many rows",
         fm_row_linear_packed(P, 16 * 65536, 512, nullptr, nullptr, 1e-5f, P, 512, 0, nullptr, nullptr, nullptr, nullptr, 0, 1, P, S), UNSUP);
  expect("pack_row_weights in place", fm_pack_row_weights(P, 512, 512, P, S), BAD);
  expect("layer_norm zero channels", fm_layer_norm(P, P, P, 4, 0, 1e-5f, P, S), BAD);
  expect("apply_rope null table", fm_apply_rope(P, 4, 1536, 1024, 64, nullptr, P, 4, S), BAD);
  expect("window_attention misaligned ld", fm_window_attention(P, 1534, 0, 512, 1024, nullptr, nullptr, 1, 250, 8, 8, 64, 250, 0.125f, P, 512, S), BAD);
  expect("window_attention_rows start past end",
         fm_window_attention_rows(P, 1536, 0, 512, 1024, nullptr, nullptr, 1, 250, 251, 8, 8, 64, 250, 0.125f, P, 512, S), BAD);
  expect("window_attention_rows nothing to do",
         fm_window_attention_rows(P, 1536, 0, 512, 1024, nullptr, nullptr, 1, 250, 250, 8, 8, 64, 250, 0.125f, P, 512, S), 0);

  // Quantizer.
  expect("rvq prepare zero entries", fm_rvq_prepare_codebook(P, P, 0, 256, 1e-5f, P, P, P, S), BAD);
  expect("rvq encode small workspace", fm_rvq_encode(P, 256, 125, 125, 256, 2048, 8, P, P, P, C, 1000, P, 16, S), WS);
  expect("rvq encode no rows", fm_rvq_encode(P, 256, 0, 125, 256, 2048, 8, P, P, P, C, 1000, nullptr, 0, S), 0);
  expect("rvq encode dim not a multiple of 4", fm_rvq_encode(P, 256, 125, 125, 250, 2048, 8, P, P, P, C, 1000, P, 1 << 30, S), BAD);
  expect("rvq split ld too small", fm_rvq_encode_split(P, 256, 125, 125, 256, 2048, 1, 7, P, P, P, C, 1000, P, 1 << 30, S), BAD);
  expect("rvq split small workspace",
         fm_rvq_encode_split(P, 512, 125, 125, 256, 2048, 1, 7, P, P, P, C, 1000, P,
                             fm_rvq_split_workspace_bytes(125, 256, 2048) - 1, S), WS);
  expect("rvq split no codebooks", fm_rvq_encode_split(P, 512, 125, 125, 256, 2048, 0, 0, P, P, P, C, 1000, P, 1 << 30, S), BAD);
  expect("rvq noalloc past the scratch",
         fm_rvq_encode_split_noalloc(P, 512, 9000, 9000, 256, 2048, 1, 7, P, P, P, C, 72000, S), SCRATCH);
  expect("rvq decode null codes", fm_rvq_decode(nullptr, 1, 8, 125, 1, P, 2048, 256, P, S), BAD);
  expect("rvq decode empty", fm_rvq_decode(C, 0, 8, 125, 1, P, 2048, 256, P, S), 0);
  expect("upsample zero kernel", fm_upsample_depthwise(P, 1, 125, 512, P, 0, 2, P, S), BAD);
  expect("linear rope null table", fm_linear_rope(P, 4000, 512, P, 1536, 64, nullptr, P, 1024, 250, P, P, 1 << 20, S), BAD);
  expect("linear rope ragged head", fm_linear_rope(P, 4000, 512, P, 1536, 64, P, P, 1000, 250, P, P, 1 << 20, S), BAD);
  expect("linear rope past the columns", fm_linear_rope(P, 4000, 512, P, 1536, 64, P, P, 1600, 250, P, P, 1 << 20, S), BAD);
  expect("linear rope FP32 weights", fm_linear_rope(P, 4000, 512, P, 1536, 0, P, P, 1024, 250, P, P, 1 << 20, S), UNSUP);
  expect("copy null source", fm_copy_buffers(nullptr, P, 16, nullptr, nullptr, 0, S), BAD);
  expect("copy null second target", fm_copy_buffers(P, P, 0, P, nullptr, 4, S), BAD);
  expect("copy nothing", fm_copy_buffers(nullptr, nullptr, 0, nullptr, nullptr, 0, S), 0);

  // Size queries at the edges of int: computed in size_t, monotone, no overflow.
  const size_t a = fm_rvq_workspace_bytes(INT_MAX, 256, 2048);
  const size_t b = fm_rvq_workspace_bytes(INT_MAX / 2, 256, 2048);
  expect("rvq workspace monotone", a > b, 1);
  expect("rvq split workspace is two branches",
         fm_rvq_split_workspace_bytes(8000, 256, 2048) == 2 * fm_rvq_workspace_bytes(8000, 256, 2048), 1);
  expect("resblock64_conv workspace grows", fm_resblock64_conv_workspace_bytes(64, INT_MAX / 64) > 0, 1);
  expect("noalloc scratch is 48 MiB", (long)fm_rvq_noalloc_scratch_bytes(), 48L << 20);
  expect("abi version", fm_abi_version(), 1);

  std::printf("%s: %d failure(s)\n", failures ? "FAILED" : "ok", failures);
  return failures ? 1 : 0;
}
