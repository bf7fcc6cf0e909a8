/*
 * mi355x_encoder.h -- C ABI of libmi355x_encoder.so, the gfx950 (MI355X)
 * implementation of the Transformer encoder forward benchmarked by
 * transformer_benchmark/models.py in the reference repository.
 *
 * Conventions shared by every entry point:
 *   - All tensors are raw device pointers owned by the caller.  The library
 *     never allocates or frees device memory and never synchronises the host,
 *     so every call is safe inside HIP graph capture.  Its only device memory
 *     is static, per GPU: the scratch array of the no-allocation forward and
 *     a 128 KiB table of the GELU of every bf16 value, which the first GELU
 *     product on a device fills with two launches on the caller's stream
 *     (recorded into the graph when that first product is captured).
 *   - bf16 tensors are passed as `void*` to 16-bit storage (IEEE bfloat16).
 *     Activations are dense row-major; weights use nn.Linear's [out, in]
 *     row-major layout, exactly as they sit in a PyTorch state_dict.
 *   - `stream` is a hipStream_t (pass torch.cuda.current_stream().cuda_stream);
 *     0 means the null stream.
 *   - Return value 0 is success.  Any other value is an error code below and
 *     enc_last_error() returns a message for the calling thread.  An
 *     out-of-memory condition reported by HIP yields ENC_ERR_OOM and a message
 *     containing "out of memory", so the reference runner's OOM classification
 *     (runner.py:502-503) still applies.
 *   - Masks are uint8 arrays (one byte per token, nonzero = valid token), the
 *     byte view of a torch.bool [batch, seq_len] tensor.
 */
#ifndef MI355X_ENCODER_H
#define MI355X_ENCODER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define ENC_OK 0
#define ENC_ERR_INVALID 1     /* bad argument: null pointer, bad size     */
#define ENC_ERR_UNSUPPORTED 2 /* shape outside what the kernels support   */
#define ENC_ERR_HIP 3         /* a HIP runtime call or launch failed      */
#define ENC_ERR_OOM 4         /* HIP reported out of memory               */

/* Epilogues of enc_linear_bf16.  y = bf16(a . weight^T + bias) always comes
 * first (fp32 accumulation, one rounding to bf16, the nn.Linear boundary). */
#define ENC_EPI_BIAS 0               /* out = y                                   */
#define ENC_EPI_BIAS_GELU 1          /* out = bf16(gelu_erf(y))                   */
#define ENC_EPI_BIAS_RESIDUAL_KEEP 2 /* out = bf16(residual + y); masked rows:
                                        out = residual                            */
#define ENC_EPI_BIAS_RESIDUAL_ZERO 3 /* out = bf16(residual + y); masked rows:
                                        out = 0                                   */

/* Library version, (major << 16) | minor. */
int enc_version(void);

/* Message of the last failed call on this thread ("" if none). */
const char* enc_last_error(void);

/* LayerNorm over the last dimension with fp32 statistics:
 *   y[r, :] = bf16(gamma * ((x[r, :] - mean) * rsqrt(var + eps)) + beta)
 * If row_mask is non-null, rows with row_mask[r] == 0 are written as zeros
 * (the masked_fill that follows final_norm).  width is a power of two in
 * [32, 4096].  The statistics follow torch's ROCm LayerNorm operation for
 * operation, so the bf16 output equals nn.LayerNorm's bit for bit.
 * Replaces nn.LayerNorm at transformer_benchmark/models.py:721,723,907 and the
 * case-6 kernel wrapper transformer_benchmark/case6_exact_layer_norm.py:98-121
 * (kernel host function case6_exact_layer_norm.cu:157-198). */
int enc_layernorm_bf16(const void* x, const void* gamma, const void* beta,
                       void* y, int64_t rows, int64_t width, float eps,
                       const uint8_t* row_mask, void* stream);

/* out[rows, out_features] = epilogue(a[rows, in_features] . weight^T + bias)
 * with bf16 MFMA and fp32 accumulation.  residual (same shape as out) is read
 * by the RESIDUAL epilogues only; row_mask (nullable, length rows) selects the
 * masked-row behaviour described at the ENC_EPI_* constants.
 * in_features % 32 == 0 and out_features % 32 == 0; rows is arbitrary.
 * Replaces nn.Linear + F.gelu + residual add at transformer_benchmark/models.py:
 * 76, 733-734 and the fused wrappers fused_ffn.py:91-126 (bias+GELU),
 * fused_ffn_out.py:89-132 (bias+residual), fused_attention_out.py:89-130
 * (out-proj+residual) and cublaslt_linear.py:292-344 (bias GEMM). */
int enc_linear_bf16(const void* a, const void* weight, const void* bias,
                    const void* residual, void* out, int64_t rows,
                    int64_t out_features, int64_t in_features, int32_t epilogue,
                    const uint8_t* row_mask, void* stream);

/* Registers, for the given device, the reduction order that the reference's
 * nn.Linear (torch.nn.functional.linear, i.e. hipBLASLt on ROCm) uses for the
 * bf16 product [rows, in_features] x [out_features, in_features]^T, as measured
 * on that device by the host.  tile_rows == 0 records that no output tile has
 * its K range split: every product of this shape (and the head-major QKV
 * projection of three such slices) accumulates K sequentially.  Otherwise the
 * library's last output tiles of 256 x 256 are a stream-K tail: split is a
 * row-major [tile_rows, tile_cols] table of the tiles from tile row
 * first_tile_row to the last (tile_cols = out_features / 256), each entry the
 * first K index of the tile's second partial sum (a multiple of 32), or 0 for
 * a tile accumulated in one pass; such a tile is computed as
 * bf16((P1 + P2) + bias), P1 over K < split and P2 over K >= split.  At most
 * 1024 entries.  A registration replaces an earlier one for the same shape
 * and device, and takes precedence over the library's built-in tables (two
 * shapes, measured on a 256-CU MI355X and used only on such a device).
 * Host-side state only; safe to call from any thread, not during a call that
 * runs the same shape.  Replaces what the reference gets implicitly from
 * hipBLASLt at every nn.Linear call (transformer_benchmark/models.py:30-33,
 * 724-725): the library picks the split per shape, so the host measures it
 * (tiktoktechjam2026track3_amd/linear_order.py) and hands it down here. */
int enc_linear_order_register(int32_t device, int64_t rows, int64_t out_features,
                              int64_t in_features, int32_t first_tile_row,
                              int32_t tile_rows, int32_t tile_cols,
                              const uint16_t* split);

/* Forgets every registered order (all devices). */
int enc_linear_order_clear(void);

/* Test hook, no counterpart in the reference (for tests that must tell the
 * GELU epilogue's two paths apart; they give the same bits by design).  On
 * the current device, enqueued on stream after the GELU table's fill:
 * ready >= 0 sets the table's ready flag (0 makes every GELU epilogue of the
 * wide GEMM evaluate the erf, 1 lets it read the table); entry in [0, 65535]
 * overwrites that bf16 pattern's table entry with value in [0, 65535], or
 * recomputes it when value is -1.  Not for production use: a changed entry
 * changes the GELU of every later product until it is restored. */
int enc_debug_gelu_table(int32_t ready, int32_t entry, int32_t value, void* stream);

/* Tile-packed copy of an nn.Linear weight W[out_features, in_features] for
 * the wide GEMM kernel: element (n, k) moves to
 *   ((n / P * (in_features / 32) + k / 32) * P + n % P) * 32 + k % 32,
 * P = 256 when out_features % 256 == 0, else 128, so each 32-deep K slice of a
 * P-row group of W is one contiguous block (one 1 KiB run per load
 * instruction instead of 64-byte pieces of rows in_features apart).  packed
 * holds out_features * in_features bf16 elements and must not alias weight;
 * out_features % 128 == 0, in_features % 32 == 0, both pointers 16-byte
 * aligned.  The copy is a pure permutation: every product computed from it is
 * bitwise the product computed from weight.  Replaces the load-time weight
 * packing of transformer_benchmark/models.py:105-158 and copy_model_weights
 * (:1242-1255) on the candidate side, whose packed [3D, D] QKV weight this
 * library takes as the plain weight; the tile layout is this library's. */
int enc_prepack_weight_bf16(const void* weight, void* packed,
                            int64_t out_features, int64_t in_features,
                            void* stream);

/* enc_linear_bf16 with the weight's tile-packed copy (enc_prepack_weight_bf16
 * of weight) beside it: the wide kernel reads packed_weight, the kernels for
 * few rows read weight; the result is bitwise that of enc_linear_bf16.
 * out_features % 128 == 0.  Same reference code as enc_linear_bf16. */
int enc_linear_prepacked_bf16(const void* a, const void* weight,
                              const void* packed_weight, const void* bias,
                              const void* residual, void* out, int64_t rows,
                              int64_t out_features, int64_t in_features,
                              int32_t epilogue, const uint8_t* row_mask,
                              void* stream);

/* The FFN half of an encoder block in one call, as the reference's block
 * computes it (models.py:724-725, 734-737):
 *   hidden = bf16(gelu_erf(bf16(h . w_in^T + b_in)))       [rows, ffn_dim]
 *   out    = bf16(residual + bf16(hidden . w_out^T + b_out)) [rows, d_model]
 * and, with row_mask non-null, out rows with row_mask[r] == 0 are zeros (the
 * block output's masked_fill).  Two MFMA GEMM launches with the GELU and the
 * residual fused into their epilogues; hidden is caller workspace of
 * rows * ffn_dim bf16 that must not overlap h, residual or out (out may
 * alias residual).  d_model and ffn_dim multiples of 32.  Bitwise the
 * encoder forward's FFN.  Replaces ffn_in / F.gelu / ffn_out + residual at
 * models.py:724-725, 734 and the candidate's fused wrappers fused_ffn.py:91-126
 * and fused_ffn_out.py:89-132. */
int enc_ffn_fused_bf16(const void* h, const void* w_in, const void* b_in,
                       const void* w_out, const void* b_out,
                       const void* residual, void* out, void* hidden,
                       int64_t rows, int64_t d_model, int64_t ffn_dim,
                       const uint8_t* row_mask, void* stream);

/* Packed QKV projection x[batch*seq_len, d_model] . qkv_weight[3*d_model,
 * d_model]^T + qkv_bias, rounded to bf16 and written head-major:
 *   q, k : [batch, num_heads, seq_len, head_dim]
 *   v_t  : [batch, num_heads, head_dim, round_up(seq_len, 8)]  (V transposed
 *          per head; the padding columns are never read)
 * head_dim = d_model / num_heads.  Replaces the packed projection and
 * .contiguous() head split of transformer_benchmark/models.py:160-240 and the
 * direct-layout wrapper direct_qkv.py:110-187 (baseline: models.py:35-53). */
int enc_qkv_proj_bf16(const void* x, const void* weight, const void* bias,
                      void* q, void* k, void* v_t, int64_t batch,
                      int64_t seq_len, int64_t d_model, int64_t num_heads,
                      void* stream);

/* Streaming attention; scores are never materialised.
 * For each (b, h, query i), over keys j that are allowed:
 *   s_ij = bf16(bf16(q_i . k_j) * scale)
 *   p_ij = bf16(softmax_j(s_ij)) in fp32 ;  context = bf16(sum_j p_ij v_j)
 * bit for bit as the reference computes them with torch on ROCm (the softmax
 * max/sum/divide follow torch's reduction order), by sweeping the keys three
 * times (row max, row sum, probabilities + P.V).  seq_len above 2048 must be
 * a multiple of 4, and one head's K (seq_len * head_dim) and V^T
 * (head_dim * round_up(seq_len, 8)) must each stay under 4 GiB (the tile
 * loads use 32-bit offsets inside a head); ENC_ERR_UNSUPPORTED otherwise.
 * Key j is excluded when causal and j > i, when kv_len is non-null and
 * j >= kv_len[b] (prefix padding), or when key_mask is non-null and
 * key_mask[b, j] == 0.  With kv_len, query rows i >= kv_len[b] are padding and
 * are written as zeros.  A query row with no allowed key is written as zeros.
 * context: [batch, seq_len, num_heads * head_dim] (token-major, the layout
 * out_proj consumes).  head_dim is 8, 32, 64, 128 or 256; v_t as produced by
 * enc_qkv_proj_bf16.
 * Replaces transformer_benchmark/models.py:55-75 (baseline) and the
 * candidate's score/softmax/PV kernels: triangular_scores.py:110-291,
 * pv_context.py:79-542, native_softmax_bf16.py:129-184,
 * case6_exact_attention.py:119-148, case13_exact_attention.py:50-77. */
int enc_attention_fwd_bf16(const void* q, const void* k, const void* v_t,
                           void* context, int64_t batch, int64_t num_heads,
                           int64_t seq_len, int64_t head_dim, float scale,
                           int32_t causal, const int32_t* kv_len,
                           const uint8_t* key_mask, void* stream);

/* One-pass attention with an online softmax: same arguments, masking and
 * layouts as enc_attention_fwd_bf16, any seq_len, head_dim 64 only.  Scores
 * are rounded as the
 * reference rounds them, but the exponentials exp(s_ij - m_i) are rounded to
 * bf16 before the division by the row sum instead of after it, so the context
 * differs from the reference's by bf16 rounding noise of the weights.  That
 * noise compounds through a deep bf16 stack past the reference's elementwise
 * gate, so the encoder uses it only when asked (ENC_FWD_ONLINE_ATTENTION).
 * Same reference code as enc_attention_fwd_bf16 (models.py:55-75). */
int enc_attention_online_fwd_bf16(const void* q, const void* k, const void* v_t,
                                  void* context, int64_t batch,
                                  int64_t num_heads, int64_t seq_len,
                                  int64_t head_dim, float scale, int32_t causal,
                                  const int32_t* kv_len,
                                  const uint8_t* key_mask, void* stream);

/* Self-check of the attention's softmax exponential (no counterpart in the
 * reference; for test suites): adds to *mismatches (a device uint32 the
 * caller zeroes) the number of float bit patterns in [lo_bits, hi_bits]
 * (non-positive floats, e.g. 0x80000000 .. 0xc2d00000 = -0 .. -104) where the
 * exact attention's inlined exp differs from the device library's expf, plus
 * those where its form with the scale 1/8 folded into the constants,
 * evaluated on 8x, differs from expf(x). */
int enc_selfcheck_expf(uint32_t lo_bits, uint32_t hi_bits, uint32_t* mismatches,
                       void* stream);

/* kv_len[b] = number of valid tokens in mask[b, :] (int32, device).  Equal to
 * the prefix length for the prefix masks built by generate_random_case
 * (transformer_benchmark/cases.py:87-97). */
int enc_mask_lengths(const uint8_t* mask, int64_t batch, int64_t seq_len,
                     int32_t* kv_len, void* stream);

/* flags of enc_encoder_forward_bf16 */
#define ENC_FWD_ONLINE_ATTENTION 1 /* one-pass online-softmax attention      */
#define ENC_FWD_SKIP_FINAL_NORM 2  /* out = last block's output: the caller
                                      runs final_norm (enc_layernorm_bf16,
                                      with row_mask), e.g. into a fresh
                                      tensor after a graph replay           */
#define ENC_FWD_PACKED_WEIGHTS 4   /* weights carries 4 * num_layers more
                                      pointers: the enc_prepack_weight_bf16
                                      copies of each layer's qkv_proj,
                                      out_proj, ffn_in and ffn_out weights  */

/* Bytes of device workspace enc_encoder_forward_bf16 needs for this shape. */
int64_t enc_encoder_workspace_bytes(int64_t batch, int64_t seq_len,
                                    int64_t d_model, int64_t num_heads,
                                    int64_t ffn_dim);

/* The whole encoder forward (num_layers blocks, then final LayerNorm):
 *   per block  x = x + attention(norm1(x)) ; x = x + ffn_out(gelu(ffn_in(norm2(x))))
 * weights: 12 * num_layers + 2 device pointers, per layer in the order
 *   norm1.weight, norm1.bias, qkv_proj.weight [3D,D], qkv_proj.bias [3D],
 *   out_proj.weight, out_proj.bias, norm2.weight, norm2.bias,
 *   ffn_in.weight [F,D], ffn_in.bias, ffn_out.weight [D,F], ffn_out.bias,
 * followed by final_norm.weight, final_norm.bias; with ENC_FWD_PACKED_WEIGHTS,
 * then per layer the packed qkv_proj, out_proj, ffn_in and ffn_out weights
 * (3*d_model, d_model and ffn_dim must then be multiples of 128).
 * Masking follows the reference: with row_mask non-null, padded rows of the
 * attention output are zero (models.py:78-79), block outputs are zeroed on
 * padded rows (models.py:736-737) and so is the final output
 * (models.py:917-918).  kv_len / key_mask are passed to the attention as in
 * enc_attention_fwd_bf16 (at most one of them non-null).  x is not modified;
 * out may not alias x or the workspace.  flags: ENC_FWD_ONLINE_ATTENTION and/or
 * ENC_FWD_SKIP_FINAL_NORM (no counterpart in the reference: it lets a graph
 * replay end at a static buffer while the final norm writes the fresh output
 * tensor the reference's graph path returns as a clone, models.py:1163-1239).
 * Replaces UserOptimizedTransformer.forward / _forward_eager
 * (transformer_benchmark/models.py:1020-1049, 1202-1239) and the block
 * forward (models.py:772-892). */
int enc_encoder_forward_bf16(const void* x, void* out, void* workspace,
                             int64_t workspace_bytes,
                             const void* const* weights, int64_t batch,
                             int64_t seq_len, int64_t d_model,
                             int64_t num_heads, int64_t ffn_dim,
                             int64_t num_layers, float eps, int32_t causal,
                             const int32_t* kv_len, const uint8_t* key_mask,
                             const uint8_t* row_mask, int32_t flags,
                             void* stream);

/* Bytes of the library-owned scratch array behind
 * enc_encoder_forward_bf16_noalloc (one array per GPU). */
#define ENC_NOALLOC_SCRATCH_BYTES (64ll * 1024 * 1024)

/* enc_encoder_forward_bf16 without a caller workspace and without any device
 * allocation: the activation buffers live in a statically sized device array
 * of ENC_NOALLOC_SCRATCH_BYTES that the library holds on every GPU it runs
 * on until the process ends.  No counterpart in the reference: it is for
 * callers that cannot allocate device memory (code under HIP graph capture
 * that must not call hipMalloc, tight serving loops, harnesses that forbid
 * allocation).  Same arguments, results and errors as
 * enc_encoder_forward_bf16 otherwise; a shape whose workspace
 * (enc_encoder_workspace_bytes) exceeds the array is rejected with
 * ENC_ERR_UNSUPPORTED before anything is launched.  Every call on one GPU
 * shares that GPU's array: calls that overlap in time on one GPU (other
 * streams or threads) race and must be serialised by the caller. */
int enc_encoder_forward_bf16_noalloc(const void* x, void* out,
                                     const void* const* weights, int64_t batch,
                                     int64_t seq_len, int64_t d_model,
                                     int64_t num_heads, int64_t ffn_dim,
                                     int64_t num_layers, float eps,
                                     int32_t causal, const int32_t* kv_len,
                                     const uint8_t* key_mask,
                                     const uint8_t* row_mask, int32_t flags,
                                     void* stream);

#ifdef __cplusplus
}
#endif

#endif /* MI355X_ENCODER_H */
