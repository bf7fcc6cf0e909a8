// Exact attention entry (head-dim dispatch), the key-mask length kernel and
// the expf self-check.  The exact attention kernel itself is a template over
// the head dim (attention_exact.h), instantiated once per head dim in
// attention_hd{8,32,64,128,256}.hip so they compile in parallel.
#include "attention_exact.h"

namespace enc {

namespace {

__global__ void __launch_bounds__(256)
mask_lengths_kernel(const uint8_t* __restrict__ mask, int64_t S, int32_t* __restrict__ kv_len) {
  const int64_t b = blockIdx.x;
  const uint8_t* row = mask + b * S;
  int count = 0;
  for (int64_t j = threadIdx.x; j < S; j += blockDim.x) count += row[j] != 0;
  __shared__ int partial[4];
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) count += __shfl_xor(count, off, kWave);
  if ((threadIdx.x % kWave) == 0) partial[threadIdx.x / kWave] = count;
  __syncthreads();
  if (threadIdx.x == 0) kv_len[b] = partial[0] + partial[1] + partial[2] + partial[3];
}

// Compares expf_nonpos with the device library's expf on every float bit
// pattern in [lo, hi] (unsigned order; pass patterns of non-positive floats),
// and the scale-folded form the short-row attention uses with its scale 1/8
// (head dim 64): expf_nonpos_scaled(8x) against expf(x).  Each mismatch of
// either form counts once.
__global__ void __launch_bounds__(256)
expf_check_kernel(uint32_t lo, uint32_t hi, uint32_t* __restrict__ mismatches) {
  const uint64_t per_block = 256ull * 64ull;
  const uint64_t first = lo + static_cast<uint64_t>(blockIdx.x) * per_block + threadIdx.x;
  const ExpfScaled eighth = expf_scaled_consts(0.125f);
  uint32_t bad = 0;
  for (int i = 0; i < 64; ++i) {
    const uint64_t bits = first + static_cast<uint64_t>(i) * 256ull;
    if (bits > hi) break;
    const float x = __uint_as_float(static_cast<uint32_t>(bits));
    const uint32_t ref = __float_as_uint(expf(x));
    bad += __float_as_uint(expf_nonpos(x)) != ref;
    bad += __float_as_uint(expf_nonpos_scaled(x * 8.0f, eighth)) != ref;
  }
  if (bad) atomicAdd(mismatches, bad);
}

}  // namespace

hipError_t expf_selfcheck(uint32_t lo_bits, uint32_t hi_bits, uint32_t* mismatches, hipStream_t stream) {
  if (hi_bits < lo_bits) return hipErrorInvalidValue;
  const uint64_t count = static_cast<uint64_t>(hi_bits) - lo_bits + 1;
  const uint64_t blocks = (count + 256ull * 64ull - 1) / (256ull * 64ull);
  hipLaunchKernelGGL(expf_check_kernel, dim3(static_cast<uint32_t>(blocks)), dim3(256), 0, stream, lo_bits,
                     hi_bits, mismatches);
  return hipGetLastError();
}

bool attention_seq_supported(int64_t seq_len, int64_t head_dim) {
  // torch's long-row softmax folds 4-element vectors; other lengths are not pinned
  if (!(seq_len <= kWarpSoftmaxMaxKeys || seq_len % 4 == 0)) return false;
  // the tile loads address one head's K and V^T with 32-bit byte offsets
  return vt_stride(seq_len) * head_dim * 2 < (int64_t(1) << 32);
}

hipError_t attention_fwd_bf16(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx,
                              int batch, int heads, int seq_len, int head_dim, float scale,
                              bool causal, const int32_t* kv_len, const uint8_t* key_mask,
                              hipStream_t stream) {
  if (batch == 0 || seq_len == 0) return hipSuccess;
  switch (head_dim) {
    case 8:
      return attention_exact_hd8(q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, causal, stream);
    case 32:
      return attention_exact_hd32(q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, causal, stream);
    case 64:
      return attention_exact_hd64(q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, causal, stream);
    case 128:
      return attention_exact_hd128(q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, causal, stream);
    case 256:
      return attention_exact_hd256(q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, causal, stream);
    default:
      return hipErrorInvalidValue;
  }
}

hipError_t mask_lengths(const uint8_t* mask, int64_t batch, int64_t seq_len, int32_t* kv_len,
                        hipStream_t stream) {
  if (batch == 0) return hipSuccess;
  hipLaunchKernelGGL(mask_lengths_kernel, dim3(static_cast<uint32_t>(batch)), dim3(256), 0, stream,
                     mask, seq_len, kv_len);
  return hipGetLastError();
}

}  // namespace enc
