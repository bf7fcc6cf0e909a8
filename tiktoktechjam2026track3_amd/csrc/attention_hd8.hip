// Exact attention kernels at head_dim 8 (the template is in attention_exact.h).
#include "attention_exact.h"

namespace enc {

hipError_t attention_exact_hd8(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx, int batch,
                                int heads, int seq_len, float scale, const int32_t* kv_len,
                                const uint8_t* key_mask, bool causal, hipStream_t stream) {
  return exact_attention<8>(q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, causal, stream);
}

}  // namespace enc
