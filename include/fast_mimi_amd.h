/*
 * fast_mimi_amd.h — C ABI of libfast_mimi_amd.so, the MI355X (gfx950) kernels
 * of the Mimi codec encode/decode hot path.
 *
 * Conventions (all entry points):
 *   - Pointers are device pointers (hipMalloc / torch CUDA tensors); sizes are
 *     element counts.  Activations are FP32, channels-last: a tensor of `batch`
 *     items, `length` positions and `channels` channels is the contiguous array
 *     [batch][length][channels].  The reference keeps NCL ([batch][channels]
 *     [length]); for 1-channel audio the two layouts coincide.
 *   - Work is enqueued on `stream`; nothing synchronizes.  Calls sharing a
 *     `workspace` must be ordered on one stream.
 *   - Return value: 0 on success, 1000 bad argument, 1001 workspace too small,
 *     1002 unsupported shape, 1003 input larger than the fixed scratch of an
 *     allocation-free entry point, otherwise the hipError_t of the launch.
 *   - Packed weights ("W^T layout") are [N][K] row-major with K contiguous:
 *       Conv1d weight [C_out][C_in][k]     -> [C_out][k * C_in], k-major:
 *                                             element (co, tap*C_in + ci) = w[co][ci][tap]
 *       ConvTranspose1d weight [C_in][C_out][k], k = taps * stride
 *                                          -> [stride * C_out][taps * C_in]:
 *                                             element (r*C_out + co, jj*C_in + ci)
 *                                             = w[ci][co][r + (taps - 1 - jj) * stride]
 *       Linear weight [out][in]            -> unchanged.
 *
 * Each entry point names the reference interface (kadirnar/fast-mimi,
 * src/fast_mimi/...) whose computation it replaces.
 */
#ifndef FAST_MIMI_AMD_H_
#define FAST_MIMI_AMD_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef struct ihipStream_t* hipStream_t;

/* Epilogue / loader flags (bit set). */
enum {
  FM_ELU_IN = 1,        /* ELU applied to the input as it is loaded            */
  FM_REPLICATE = 2,     /* internal: replicate padding (use pad_mode = 1)      */
  FM_EPI_ELU = 4,       /* ELU on the output                                   */
  FM_EPI_GELU = 8,      /* exact-erf GELU on the output                        */
  FM_EPI_RES_ADD = 16,  /* y = residual + (acc + bias)                         */
  FM_EPI_RES_SCALE = 32, /* y = residual + scale[n] * acc   (fm_linear only)    */
  FM_WEIGHTS_X6 = 64,    /* weight is followed by its bf16 planes (fm_split_weights) */
  FM_ACT_EXP = 128       /* residual blocks: ELU as e^x - 1 (see fm_resblock)     */
};

/* ABI version of the library (bumped when a contract changes). */
int fm_abi_version(void);

/*
 * Diagnostics (no counterpart in the reference, which has no kernel
 * selection of its own to report): writes into `buf` (at most `size` bytes,
 * NUL-terminated) the kernel instantiation, tile count and K-split count that
 * the last fm_conv1d / fm_conv1d_valid / fm_conv_transpose1d / fm_linear call
 * made on the calling host thread launched ("" before any).  Host only.
 */
int fm_gemm_last_plan(char* buf, int size);

/*
 * bf16x6 weights: writes the three round-to-nearest bf16 pieces of each
 * float of a packed weight W^T [rows][cols] (cols a multiple of 16, else
 * FM_UNSUPPORTED) into `planes` in k16-tile order [3][cols/16][rows][16].
 * A caller that stores the planes directly after the FP32 weight (one buffer
 * of rows * cols * 10 bytes) and adds FM_WEIGHTS_X6 (64) to `flags` of
 * fm_conv1d / fm_conv1d_valid / fm_conv_transpose1d / fm_linear (or to
 * `elu_out` of fm_resblock, both weights split) lets the large tiles and the
 * C = 128 / 256 residual blocks run the FP32 contraction as six bf16 MFMA
 * products per operand pair (FP32-accurate, see csrc/fm_gemm.hip); every
 * other kernel reads the FP32 part only.
 * No reference counterpart: it prepares the operands of the convolutions the
 * entry points below replace.
 */
int fm_split_weights(const float* weight_packed, int rows, int cols, void* planes, hipStream_t stream);

/*
 * Causal Conv1d, dilation 1: left zero (pad_mode 0) or edge (pad_mode 1)
 * padding of kernel - stride, right padding to a multiple of the stride;
 * output length ceil(length / stride), of which the first y_length rows per
 * batch item are written (y is [batch][y_length][out_channels]).
 * Replaces MimiConv1d.forward + _pad1d + _get_extra_padding_for_conv1d
 * (model.py:697-797) and the cuDNN exact encoder convs (_optimized_runtime.py:937-1218).
 * workspace: optional scratch for K-split partial sums (may be NULL).
 */
int fm_conv1d(const float* x, int batch, int length, int in_channels, const float* weight_packed,
              const float* bias, int out_channels, int kernel, int stride, int pad_mode, int flags,
              const float* residual, float* y, int y_length, float* workspace,
              size_t workspace_bytes, hipStream_t stream);

/*
 * fm_conv1d for few output rows and long K (the 12.5-25 Hz end of the SEANet
 * stacks at batch x rows <= a few hundred): same padding, output length and
 * arithmetic contract, but every 16 output rows x 32 columns is one block
 * whose 8 waves split K, so there is no K-split partial buffer and no second
 * launch.  weight is the conv's W^T [out_channels][kernel * in_channels],
 * either in fm_pack_row_weights order (FP32 MFMA) or, with FM_WEIGHTS_X6 in
 * flags, the plain W^T followed by its fm_split_weights planes (bf16x6).
 * bias[n % bias_len] is added to output column n.  flags: FM_ELU_IN,
 * FM_EPI_ELU, FM_EPI_RES_ADD (residual shaped as y), FM_WEIGHTS_X6; y is
 * [batch][ceil(length / stride)][out_channels].
 * A causal ConvTranspose1d of stride s and kernel taps * s is this call with
 * kernel taps, stride 1, out_channels s * c_out (its phase-major W^T) and
 * bias_len c_out: y is then [batch][length * s][c_out].
 * Shapes: fm_conv1d_rows_supported(in, out, kernel, flags) != 0 (out_channels
 * a multiple of 32; in_channels * kernel 1536, 2048, 3072 or 3584 with
 * in_channels a multiple of 64, or with FM_WEIGHTS_X6 also 256 and
 * in_channels a multiple of 32), else FM_UNSUPPORTED.  Replaces
 * MimiConv1d.forward (model.py:697-797) at those shapes: the encoder's last
 * conv, the replicate-padded downsample (model.py:2730-2741), the decoder's
 * first conv and the 512-channel residual blocks' two convs.
 */
int fm_conv1d_rows_supported(int in_channels, int out_channels, int kernel, int flags);
int fm_conv1d_rows(const float* x, int batch, int length, int in_channels, const float* weight,
                   const float* bias, int bias_len, int out_channels, int kernel, int stride,
                   int pad_mode, int flags, const float* residual, float* y, hipStream_t stream);

/*
 * Conv1d over exactly the given rows, no padding: output row t reads input
 * rows t*stride .. t*stride + kernel - 1; y is [batch][(length - kernel) /
 * stride + 1][out_channels].  Streaming convolution: the caller prepends the
 * layer's cached left context.  Replaces MimiConv1d.forward with a padding
 * cache (model.py:764-797, MimiConv1dPaddingCache.update :536-620).
 */
int fm_conv1d_valid(const float* x, int batch, int length, int in_channels,
                    const float* weight_packed, const float* bias, int out_channels, int kernel,
                    int stride, int flags, const float* residual, float* y, float* workspace,
                    size_t workspace_bytes, hipStream_t stream);

/*
 * Causal ConvTranspose1d with the full right trim (trim ratio 1): output
 * [batch][length * stride][out_channels].  kernel must be a multiple of stride.
 * Replaces MimiConvTranspose1d.forward (model.py:886-897),
 * mimi_cutlass_bias_dgrad (cutlass_bias_dgrad.cu:147-157) and the cuDNN
 * deconvolutions (_optimized_runtime.py:571-753).
 */
int fm_conv_transpose1d(const float* x, int batch, int length, int in_channels,
                        const float* weight_packed, const float* bias, int out_channels, int kernel,
                        int stride, int flags, const float* residual, float* y, float* workspace,
                        size_t workspace_bytes, hipStream_t stream);

/*
 * y[rows][out] = epilogue(x[rows][in] . W^T), no bias.  residual/scale feed
 * FM_EPI_RES_SCALE (LayerScale residual; y may alias residual).
 * Replaces the nn.Linear projections of MimiAttention / MimiMLP
 * (model.py:1870-1961, :1990-1999), the RVQ 1x1 in/out projections
 * (model.py:2408-2444) and _packed_qkv.py:139-150.
 */
int fm_linear(const float* x, int rows, int in_features, const float* weight_packed,
              int out_features, int flags, const float* residual, const float* scale, float* y,
              float* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Fused SEANet residual block: y = ELU?(x + conv1x1(ELU(conv_k3(ELU(x))))),
 * hidden width channels/2, x and y [batch][length][channels], x != y.
 * Supported widths: fm_resblock_supported(channels) != 0.
 * Replaces MimiResnetBlock.forward (model.py:947-971), decoder9_fused_wmma
 * (decoder9_fused_wmma.cu:87-112) and the Triton _add_elu_half_kernel
 * (_optimized_runtime.py:37-77).
 */
int fm_resblock_supported(int channels);
int fm_resblock(const float* x, int batch, int length, int channels, const float* w1_packed,
                const float* b1, const float* w2_packed, const float* b2, int elu_out, float* y,
                hipStream_t stream);
/* elu_out: nonzero (other than the FM_WEIGHTS_X6 and FM_ACT_EXP bits)
 * applies the trailing ELU; FM_WEIGHTS_X6 says both packed weights carry
 * their fm_split_weights planes (the block then runs on the bf16 matrix
 * cores).  FM_ACT_EXP (with FM_WEIGHTS_X6) evaluates the block's ELUs as
 * e^x - 1 from the hardware exponential: about half the vector instructions,
 * an absolute error of a few 1e-8 near zero instead of a relative one.  For
 * callers held to an absolute bar (the decoder's waveform), not for the
 * encoder, whose codes depend on exact activations. */

/*
 * The SEANet encoder's first conv (1 -> 64 channels, kernel 7, causal, no
 * activation) fused into the 64-channel residual block after it:
 * y = fm_resblock(conv(wav)), wav [batch][length], y [batch][length][64].
 * w0_packed is the conv's packed [64][7] weight.  The 64-channel conv output
 * is formed on chip and never stored.
 * Replaces MimiEncoder layers.0 + layers.1 (model.py:1013-1031).
 * elu_out may carry FM_WEIGHTS_X6 and FM_ACT_EXP as in fm_resblock.
 */
int fm_conv_resblock64(const float* wav, int batch, int length, const float* w0_packed,
                       const float* b0, const float* w1_packed, const float* b1,
                       const float* w2_packed, const float* b2, int elu_out, float* y,
                       hipStream_t stream);

/*
 * The SEANet decoder's last 64-channel residual block (ELU after it when
 * elu_mid != 0) fused with the waveform conv after it (64 -> 1 channel,
 * kernel 3, causal): out[b][t] = b3 + sum_j w3[j] . block(x)[b][t-2+j] for
 * t < y_len, out [batch][y_len].  w3_packed is the conv's packed [3][64]
 * weight (b3 may be NULL).  The 64-channel block output is reduced on chip
 * to three tap products per row (the workspace,
 * fm_resblock64_conv_workspace_bytes) and never stored.
 * Replaces MimiDecoder's last MimiResnetBlock + ELU + MimiConv1d
 * (model.py:1269-1285).
 */
/* elu_mid may carry FM_WEIGHTS_X6 and FM_ACT_EXP as in fm_resblock. */
size_t fm_resblock64_conv_workspace_bytes(int batch, int length);
int fm_resblock64_conv(const float* x, int batch, int length, const float* w1_packed,
                       const float* b1, const float* w2_packed, const float* b2, int elu_mid,
                       const float* w3_packed, const float* b3, int y_len, float* out,
                       float* workspace, size_t workspace_bytes, hipStream_t stream);

/*
 * Transformer projection y[rows][out] = epilogue(LN?(x) . W^T), no bias:
 *   - ln_gamma/ln_beta non-NULL: x rows are layer-normalised (biased variance,
 *     eps ln_eps) inside the kernel first;
 *   - rope_cos/rope_sin non-NULL ([rows_per_seq][64] tables): columns below
 *     rope_cols (a multiple of 64) get RoPE per 64-wide head, position
 *     row % rows_per_seq;
 *   - flags: FM_EPI_GELU, or FM_EPI_RES_SCALE (y = residual + scale[n] * acc,
 *     y may alias residual); with FM_WEIGHTS_X6 the weight is followed by its
 *     fm_split_weights planes and 16-row blocks run the contraction on the
 *     bf16 matrix cores (bf16x6, FP32-accurate).
 * Supported shapes: fm_row_linear_supported(in, out) != 0 (in 512 or 2048,
 * out a multiple of 64; LayerNorm and RoPE only with in == 512).  Replaces the LayerNorm + q/k/v projection + _apply_rope
 * and LayerNorm + fc1 + GELU sequences of MimiTransformerLayer
 * (model.py:2028-2061, :1870-1961, :1551-1569, :1990-1999) and the Triton
 * _packed_qkv_rope_kernel (_packed_qkv.py:14-131); with in == 2048 the fc2
 * projection of MimiMLP (model.py:1990-1999); also fits the RVQ 1x1
 * projections (model.py:2408-2444).
 */
int fm_row_linear_supported(int in_features, int out_features);
int fm_row_linear(const float* x, int rows, int in_features, const float* ln_gamma,
                  const float* ln_beta, float ln_eps, const float* weight, int out_features,
                  int flags, const float* residual, const float* scale, const float* rope_cos,
                  const float* rope_sin, int rope_cols, int rows_per_seq, float* y,
                  hipStream_t stream);

/*
 * fm_row_linear on fragment-packed weights, for few rows (16-row blocks on
 * the 16x16x4 FP32 MFMA; the choice for rows <= ~512).  Same arguments,
 * shapes and epilogues as fm_row_linear; weight_packed is produced by
 * fm_pack_row_weights.  Packed layout: the float4 at index
 * ((nt * (in/64) + kp) * 4 + t) * 64 + lane holds
 * W[16 nt + lane % 16][64 kp + 16 (lane / 16) + 4 t .. 4 t + 3].
 * Replaces the same reference computations as fm_row_linear.
 */
int fm_row_linear_packed(const float* x, int rows, int in_features, const float* ln_gamma,
                         const float* ln_beta, float ln_eps, const float* weight_packed,
                         int out_features, int flags, const float* residual, const float* scale,
                         const float* rope_cos, const float* rope_sin, int rope_cols,
                         int rows_per_seq, float* y, hipStream_t stream);
/*
 * fm_row_linear_packed (no LayerNorm, RoPE or epilogue; in_features 512,
 * out_features a multiple of 32) followed by the depthwise causal
 * ConvTranspose1d of kernel 4 and stride 2 (up_weight [out_features][4], the
 * reference's [channels][1][4]), in one launch: y is [rows * 2][out_features],
 * y[2t + p] = h[t-1] * w[p+2] + h[t] * w[p] with h[t-1] = 0 at the start of
 * each sequence of rows_per_seq rows, rounded as fm_upsample_depthwise.
 * Replaces the RVQ output projection and the bottleneck upsample of the
 * decoder (model.py:2570-2627 output_proj, :2744-2752).
 */
int fm_row_linear_packed_upsample(const float* x, int rows, int in_features,
                                  const float* weight_packed, int out_features, int rows_per_seq,
                                  const float* up_weight, float* y, hipStream_t stream);

/* Packs a [out_features][in_features] weight (out % 16 == 0, in % 64 == 0);
 * out must not alias weight.  One-time preparation, like the reference's
 * weight packing in _optimized_runtime.py / _packed_qkv.py. */
int fm_pack_row_weights(const float* weight, int out_features, int in_features, float* out,
                        hipStream_t stream);

/*
 * fm_linear (no residual, no other epilogue) with RoPE applied in the
 * epilogue: output columns 0 .. rope_cols-1 form heads of 64 columns, and
 * column d of a head at row position t = row % rows_per_seq becomes
 * y[d] * cos[t][d] - y[d + 32] * sin[t][d] (d < 32) or
 * y[d] * cos[t][d] + y[d - 32] * sin[t][d] (d >= 32), each product and the
 * sum rounded separately, as fm_apply_rope.  cos/sin tables [*][64].
 * flags must be FM_WEIGHTS_X6 (weights with planes); out_features and
 * rope_cols multiples of 64.  Equal, bit for bit, to fm_linear followed by
 * fm_apply_rope: one launch when fm_linear's plan is an unsplit bf16x6 tile
 * (RoPE in its epilogue), else that plan and then fm_apply_rope.
 * Replaces the q / k projections of MimiAttention with _apply_rope
 * (model.py:1870-1961, :1551-1569).
 */
int fm_linear_rope(const float* x, int rows, int in_features, const float* weight_packed,
                   int out_features, int flags, const float* cos_table, const float* sin_table,
                   int rope_cols, int rows_per_seq, float* y, float* workspace,
                   size_t workspace_bytes, hipStream_t stream);

/*
 * In-place RoPE on columns 0 .. rope_cols-1 of each row (heads of head_dim;
 * position row % rows_per_seq into the [*, head_dim] cos/sin tables), for
 * projections computed without fm_row_linear's fused epilogue (e.g. cached
 * transformer steps at other widths).  Replaces _apply_rope (model.py:1551-1569).
 */
int fm_apply_rope(float* x, long rows, int ld, int rope_cols, int head_dim, const float* cos_table,
                  const float* sin_table, int rows_per_seq, hipStream_t stream);

/*
 * LayerNorm over the last dimension (biased variance).
 * Replaces nn.LayerNorm in MimiTransformerLayer (model.py:2028-2061).
 */
int fm_layer_norm(const float* x, const float* gamma, const float* beta, long rows, int channels,
                  float eps, float* y, hipStream_t stream);

/*
 * Causal sliding-window attention with RoPE: q, k, v are read from the
 * packed projection qkv ([batch*length][ld_qkv], head h of q at column
 * q_offset + h*head_dim, likewise k / v with kv_heads heads); cos/sin tables
 * are [length][head_dim]; with both tables NULL, q and k are taken as already
 * rotated (e.g. by fm_row_linear's RoPE epilogue).  Key k is visible from query q iff
 * q - window < k <= q.  out is [batch*length][ld_out], head h at h*head_dim.
 * head_dim in {8, 16, 32, 64}; ld_qkv and the offsets are multiples of 4.
 * Replaces _apply_rope + F.scaled_dot_product_attention / the eager path of
 * MimiAttention.forward (model.py:1551-1569, :1870-1961), _attention_mask
 * (model.py:1627-1688), _native_window_attention (model.py:1589-1624), the
 * Triton _rope_kernel / _packed_qkv_rope_kernel / _attention_pack_nlc_kernel
 * (_optimized_runtime.py:80-258, _packed_qkv.py:14-131).
 */
int fm_window_attention(const float* qkv, int ld_qkv, int q_offset, int k_offset, int v_offset,
                        const float* cos_table, const float* sin_table, int batch, int length,
                        int heads, int kv_heads, int head_dim, int window, float scale, float* out,
                        int ld_out, hipStream_t stream);

/*
 * fm_window_attention for the queries at rows query_start .. length-1 of each
 * sequence; every row 0 .. length-1 is a key/value, so rows before
 * query_start act as a KV cache.  out holds length - query_start rows per
 * sequence.  Replaces the cached path of MimiAttention.forward with a
 * MimiKVCache (model.py:1912-1914, :363-518, mask :1627-1688).
 */
int fm_window_attention_rows(const float* qkv, int ld_qkv, int q_offset, int k_offset,
                             int v_offset, const float* cos_table, const float* sin_table,
                             int batch, int length, int query_start, int heads, int kv_heads,
                             int head_dim, int window, float scale, float* out, int ld_out,
                             hipStream_t stream);

/*
 * Codebook preparation: embed = embed_sum / max(cluster_usage, eps), its
 * transpose [dim][entries] and squared norms [entries].
 * Replaces MimiEuclideanCodebook.embed (model.py:2263-2275).
 */
int fm_rvq_prepare_codebook(const float* embed_sum, const float* cluster_usage, int entries,
                            int dim, float eps, float* embed, float* embed_t, float* norms,
                            hipStream_t stream);

/* Bytes of workspace fm_rvq_encode needs for `rows` query rows. */
size_t fm_rvq_workspace_bytes(int rows, int dim, int entries);

/*
 * Residual VQ encode of one branch: for codebooks 0..count-1 in order,
 * code = argmin_e sqrt(max(|x|^2 + |e|^2 - 2 x.e, 0)) (lowest index on ties),
 * x -= embed[code].  x rows have pitch ld_x; dim a multiple of 4.
 * Codes are int64, row (b, t) of codebook j at
 * codes[b * batch_stride + j * rows_per_batch + t].
 * embeds / embeds_t / norms: the branch's codebooks, contiguous per codebook.
 * Replaces MimiResidualVectorQuantizer.encode + MimiEuclideanCodebook.quantize
 * (model.py:2277-2291, :2408-2428) and the compiled RVQ encode.
 */
int fm_rvq_encode(const float* x, int ld_x, int rows, int rows_per_batch, int dim, int entries,
                  int count, const float* embeds, const float* embeds_t, const float* norms,
                  int64_t* codes, int batch_stride, void* workspace, size_t workspace_bytes,
                  hipStream_t stream);

/* Bytes of workspace fm_rvq_encode_split needs (two branches' worth). */
size_t fm_rvq_split_workspace_bytes(int rows, int dim, int entries);

/*
 * Split residual VQ encode: the semantic branch (codebooks 0..n_semantic-1,
 * input columns [0, dim) of x) and the acoustic branch (the next n_acoustic
 * codebooks, input columns [dim, 2*dim)) with the per-codebook rule of
 * fm_rvq_encode.  The two chains share launches (step s of both branches in
 * one grid), so the semantic chain adds no launches of its own.  ld_x >=
 * 2*dim; embeds / embeds_t / norms hold all n_semantic + n_acoustic
 * codebooks contiguously; codebook j's codes land at
 * codes[b * batch_stride + j * rows_per_batch + t].
 * Up to 128 rows at dim 256 the whole chain is one persistent launch whose
 * blocks wait on each other: two such calls must not run concurrently on one
 * GPU (different streams); one stream, or stream-ordered calls, are fine.
 * Replaces MimiSplitResidualVectorQuantizer._encode_eager (model.py:2485-2501).
 */
int fm_rvq_encode_split(const float* x, int ld_x, int rows, int rows_per_batch, int dim, int entries,
                        int n_semantic, int n_acoustic, const float* embeds, const float* embeds_t,
                        const float* norms, int64_t* codes, int batch_stride, void* workspace,
                        size_t workspace_bytes, hipStream_t stream);

/*
 * fm_rvq_encode_split without a workspace argument: it allocates nothing.
 * No counterpart in the reference; it is for callers that cannot allocate
 * (code under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc).  The step partials and residuals live in a fixed device array of
 * fm_rvq_noalloc_scratch_bytes() bytes (48 MiB: up to 8,190 rows of 256-dim
 * codebooks) that each GPU holds until the process ends.  Larger inputs
 * return 1003 (scratch limit).  All calls on one GPU share its array: calls
 * that overlap on one GPU race, so the caller serialises them.  Same
 * arguments, codes and rounding as fm_rvq_encode_split otherwise.
 */
size_t fm_rvq_noalloc_scratch_bytes(void);
int fm_rvq_encode_split_noalloc(const float* x, int ld_x, int rows, int rows_per_batch, int dim,
                                int entries, int n_semantic, int n_acoustic, const float* embeds,
                                const float* embeds_t, const float* norms, int64_t* codes,
                                int batch_stride, hipStream_t stream);

/*
 * Split-RVQ decode gather-sum: out[(b*frames + t)][0:dim] = 0 + E_0[c_0]
 * (the num_semantic first codebooks summed left to right),
 * out[...][dim:2*dim] = 0 + E_s[c_s] + E_{s+1}[c_{s+1}] + ... left to right.
 * codes int64 [batch][num_codebooks][frames]; embeds [num_codebooks][entries][dim].
 * Out-of-range codes produce NaN.
 * Replaces launch_split_rvq_decode_q32 (_cuda_rvq.py:77-89) and
 * MimiResidualVectorQuantizer.decode (model.py:2430-2444).
 */
int fm_rvq_decode(const int64_t* codes, int batch, int num_codebooks, int frames,
                  int num_semantic, const float* embeds, int entries, int dim, float* out,
                  hipStream_t stream);

/*
 * Depthwise causal ConvTranspose1d (groups == channels), right-trimmed to
 * length * stride; weight is the reference [channels][1][kernel].
 * Replaces the bottleneck upsample (model.py:2744-2752).
 */
int fm_upsample_depthwise(const float* x, int batch, int length, int channels,
                          const float* weight, int kernel, int stride, float* y,
                          hipStream_t stream);

/*
 * Copies bytes0 bytes from src0 to dst0 and bytes1 from src1 to dst1 (device
 * memory, buffers not overlapping; a zero size skips its pair) in one launch
 * on `stream`.  No reference counterpart: the hipGraph runner uses it to move
 * a call's input into the graph's static buffer and the graph's outputs into
 * caller-owned tensors, one launch for what would otherwise be one copy
 * launch per tensor (the role of the tensor copies around
 * _MimiCudaGraphRunner.replay, model.py:322-343).
 */
int fm_copy_buffers(const void* src0, void* dst0, size_t bytes0, const void* src1, void* dst1,
                    size_t bytes1, hipStream_t stream);

#ifdef __cplusplus
}
#endif

#endif /* FAST_MIMI_AMD_H_ */
