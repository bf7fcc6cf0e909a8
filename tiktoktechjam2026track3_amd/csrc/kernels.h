// Internal launchers shared between the kernel files and the C ABI.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "common.h"

namespace enc {

// Epilogue selectors of the GEMM kernel (values 0..3 mirror ENC_EPI_*).
enum Epilogue : int {
  kEpiBias = 0,
  kEpiBiasGelu = 1,
  kEpiResidualKeep = 2,
  kEpiResidualZero = 3,
  kEpiQkvHeadMajor = 4,
};

struct GemmEpilogueArgs {
  const bf16_t* bias = nullptr;      // [N]
  const bf16_t* residual = nullptr;  // [M, N]
  const uint8_t* row_mask = nullptr; // [M] or null
  bf16_t* out = nullptr;             // [M, N] row-major
  // head-major QKV outputs (kEpiQkvHeadMajor only)
  bf16_t* q = nullptr;   // [B, H, S, hd]
  bf16_t* k = nullptr;   // [B, H, S, hd]
  bf16_t* v_t = nullptr; // [B, H, hd, ld_vt]
  int seq_len = 0;
  int num_heads = 0;
  int head_dim = 0;
  int d_model = 0;
  int ld_vt = 0;
  // Optional tile-packed copy of W (gemm_prepack_weight), read by the wide
  // kernel in place of W; the other kernels read W.
  const bf16_t* w_packed = nullptr;
  int w_packed_rows = 0;  // its row-group height PN (gemm_prepack_rows)
};

// LayerNorm
bool layernorm_supported(int64_t width);
hipError_t layernorm_bf16(const bf16_t* x, const bf16_t* gamma, const bf16_t* beta, bf16_t* y,
                          int64_t rows, int64_t width, float eps, const uint8_t* row_mask,
                          hipStream_t stream);

// GEMM: C[M, N] = A[M, K] . W[N, K]^T with the given epilogue.
// Requirements: N % 32 == 0, K % 32 == 0, M >= 0.
bool gemm_supported(int64_t M, int64_t N, int64_t K);
hipError_t gemm_bf16(const bf16_t* A, const bf16_t* W, int64_t M, int64_t N, int64_t K,
                     int epilogue, const GemmEpilogueArgs& ep, int num_cus, hipStream_t stream);

// Tile-packed weight layout for the wide kernel: W[N, K] (nn.Linear layout)
// as [N / PN][K / 32][PN][32], i.e. element (n, k) at
//   ((n / PN * (K / 32) + k / 32) * PN + n % PN) * 32 + k % 32,
// so every 32-deep K stage of a PN-row group (and of any 128-row half of it)
// is one contiguous block.  gemm_prepack_rows returns PN (256 when N % 256 ==
// 0, else 128 when N % 128 == 0) or 0 when the shape has no packed form.
int gemm_prepack_rows(int64_t N, int64_t K);
hipError_t gemm_prepack_weight(const bf16_t* W, bf16_t* packed, int64_t N, int64_t K, hipStream_t stream);

// Measured reduction orders of the reference's nn.Linear (hipBLASLt) for the
// current device, keyed by the library product's (M, N, K): tile_rows == 0
// records that no tile's K range is split; otherwise split[] is a tail table
// of tile_rows x tile_cols 256 x 256 tiles from first_tile_row (first K index
// of the second partial sum, 0 for a one-pass tile).  Returns 0, or 1 when
// the table is inconsistent with the shape.
int gemm_order_register(int device, int64_t M, int64_t N, int64_t K, int first_tile_row, int tile_rows,
                        int tile_cols, const uint16_t* split);
void gemm_order_clear();
// Whether gemm_bf16 would accumulate some tile of this product in two partials.
bool gemm_has_split_tail(int64_t M, int64_t N, int64_t K, int num_cus);

// Test hook for the wide kernel's GELU table: ready >= 0 sets the device's
// ready flag (0: every GELU epilogue evaluates the erf); entry >= 0
// overwrites that table entry with value, or recomputes it when value < 0.
hipError_t gemm_debug_gelu_table(int32_t ready, int32_t entry, int32_t value, hipStream_t stream);

// Tile shape the dispatcher picks for (M, N) on a device with num_cus CUs.
void gemm_pick_tile(int64_t M, int64_t N, int epilogue, int num_cus, int* bm, int* bn);
// K-split reduction order matching torch.nn.functional.linear for this shape:
// split == 1 means sequential K; otherwise chunk-wide K chunks are accumulated
// into partial (chunk index % split) and the partials are added in order.
void gemm_split_plan(int64_t M, int64_t N, int64_t K, int* split, int* chunk);

// Exact three-sweep attention (head_dim 8, 32, 64, 128 or 256), bit-exact with the
// reference's materialised softmax.  v_t row stride is ld_vt = round_up(S, 8).
hipError_t attention_fwd_bf16(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx,
                              int batch, int heads, int seq_len, int head_dim, float scale,
                              bool causal, const int32_t* kv_len, const uint8_t* key_mask,
                              hipStream_t stream);
// The per-head-dim instantiations behind attention_fwd_bf16.
hipError_t attention_exact_hd8(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx, int batch,
                               int heads, int seq_len, float scale, const int32_t* kv_len,
                               const uint8_t* key_mask, bool causal, hipStream_t stream);
hipError_t attention_exact_hd32(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx, int batch,
                                int heads, int seq_len, float scale, const int32_t* kv_len,
                                const uint8_t* key_mask, bool causal, hipStream_t stream);
hipError_t attention_exact_hd64(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx, int batch,
                                int heads, int seq_len, float scale, const int32_t* kv_len,
                                const uint8_t* key_mask, bool causal, hipStream_t stream);
hipError_t attention_exact_hd128(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx, int batch,
                                 int heads, int seq_len, float scale, const int32_t* kv_len,
                                 const uint8_t* key_mask, bool causal, hipStream_t stream);
hipError_t attention_exact_hd256(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx, int batch,
                                 int heads, int seq_len, float scale, const int32_t* kv_len,
                                 const uint8_t* key_mask, bool causal, hipStream_t stream);

// Online-softmax attention (one pass over the keys), head_dim 64; same
// arguments and masking rules as attention_fwd_bf16.
hipError_t flash_attention_fwd_bf16(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx,
                                    int batch, int heads, int seq_len, int head_dim, float scale,
                                    bool causal, const int32_t* kv_len, const uint8_t* key_mask,
                                    hipStream_t stream);

// Fused block tail for d_model and ffn_dim of 32, 64 or 128: out_proj +
// residual (rows masked out keep x), norm2, ffn_in + GELU, ffn_out + residual
// (rows masked out become 0), bitwise the same as the four separate launches.
struct BlockTailArgs {
  const bf16_t* ctx = nullptr;  // attention context [T, D]
  const bf16_t* x = nullptr;    // block input (residual) [T, D]
  const bf16_t* wo = nullptr;   // out_proj weight [D, D] and bias [D]
  const bf16_t* bo = nullptr;
  const bf16_t* g2 = nullptr;   // norm2 weight and bias [D]
  const bf16_t* be2 = nullptr;
  const bf16_t* w1 = nullptr;   // ffn_in weight [F, D] and bias [F]
  const bf16_t* b1 = nullptr;
  const bf16_t* w2 = nullptr;   // ffn_out weight [D, F] and bias [D]
  const bf16_t* b2 = nullptr;
  bf16_t* out = nullptr;        // block output [T, D]; must not alias x (rejected)
  const uint8_t* row_mask = nullptr;
  // optional: the next layer's norm1 (weight, bias) applied to the block
  // output, written to ln_out [T, D] (no row mask, as the separate launch)
  const bf16_t* g1n = nullptr;
  const bf16_t* be1n = nullptr;
  bf16_t* ln_out = nullptr;
};
bool block_tail_supported(int64_t d_model, int64_t ffn_dim);
hipError_t block_tail_bf16(const BlockTailArgs& args, int64_t rows, int64_t d_model, int64_t ffn_dim, float eps,
                           int num_cus, hipStream_t stream);

// Sequence lengths whose softmax summation order is reproduced exactly, and
// whose per-head K and V^T the exact kernel's 32-bit tile offsets reach.
bool attention_seq_supported(int64_t seq_len, int64_t head_dim);

// Counts (atomically, into *mismatches) the float bit patterns in
// [lo_bits, hi_bits] where the attention's expf_nonpos differs from expf.
hipError_t expf_selfcheck(uint32_t lo_bits, uint32_t hi_bits, uint32_t* mismatches, hipStream_t stream);

hipError_t mask_lengths(const uint8_t* mask, int64_t batch, int64_t seq_len, int32_t* kv_len,
                        hipStream_t stream);

inline int64_t vt_stride(int64_t seq_len) { return (seq_len + 7) / 8 * 8; }

}  // namespace enc
