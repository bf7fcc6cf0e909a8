// Streaming multi-head attention forward for gfx950, head_dim = 64.
//
// Scores are never materialised: each workgroup owns BQ = 128 query rows of one
// (batch, head) and streams 64-key tiles of K (and V^T) through LDS.
//
// Both products put the query index on the MFMA N dimension (the lane index),
// so every per-query quantity lives in the lane that owns that query:
//   S^T[key, q]  = K[key, :] . Q[q, :]        A = K tile (LDS), B = Q (registers)
//   O^T[d, q]   += V^T[d, key] . P^T[key, q]  A = V^T tile (LDS), B = P (registers)
// With the 32x32x16 accumulator layout (col = lane%32, row = 8*(r/4) + 4*(lane/32)
// + r%4), lane l holds query l%32 and keys {8i + 4(l/32) + j}.  Those scores are
// fed straight back as the B operand of the PV product: the MFMA reduction index
// k is mapped to keys by the same permutation, so the V^T operand reads keys
// {16kk + 4(l/32) + j} and {16kk + 8 + 4(l/32) + j} (two 8-byte LDS reads).
// V arrives transposed ([B, H, hd, S]) from the QKV projection epilogue.
//
// Numerics reproduce the reference forward (transformer_benchmark/models.py:55-70)
// rounding for rounding:
//   s = bf16(bf16(q.k) * scale)          (the second rounding is exact for 1/8)
//   p = bf16(exp(s - max_j s) / sum_j exp(s - max_j s))   fp32 softmax, then bf16
//   context = bf16(sum_j p_j v_j)        fp32 accumulation in key order
// Because p is rounded only after normalisation, the softmax takes two passes
// over the keys: pass 1 streams K and computes each row's max and sum; pass 2
// streams K and V^T, recomputes the scores, forms the final bf16 probabilities
// and accumulates PV with no rescaling.  (A one-pass online softmax rounds
// un-normalised probabilities instead, which changes almost every probability's
// rounding and, through the residual stream, moves outputs past the bf16 gate.)
//
// Tile skipping: with causal masking a workgroup stops at the last key tile its
// last query can see, and a wavefront skips the MFMAs of tiles entirely in its
// future; with prefix padding (kv_len) key tiles past kv_len are never loaded
// and query tiles past kv_len are written as zeros without any work.
#include "common.h"
#include "kernels.h"

namespace enc {

namespace {

constexpr int kHd = 64;
constexpr int kBQ = 128;   // queries per workgroup (32 per wavefront)
constexpr int kBKV = 64;   // keys per tile
constexpr int kLds = 64 + 8;  // padded LDS row (elements)
constexpr int kThreads = 256;
constexpr float kLog2e = 1.4426950408889634f;

enum MaskMode : int { kMaskNone = 0, kMaskPrefix = 1, kMaskBytes = 2 };

template <bool CAUSAL, int MASK, bool POW2_SCALE>
__global__ void __launch_bounds__(kThreads)
attn_fwd_hd64_kernel(const bf16_t* __restrict__ Q, const bf16_t* __restrict__ Kg,
                     const bf16_t* __restrict__ Vt, bf16_t* __restrict__ ctx, int H, int S,
                     int ld_vt, int num_qblocks, float scale,
                     const int32_t* __restrict__ kv_len, const uint8_t* __restrict__ key_mask) {
  __shared__ __attribute__((aligned(16))) bf16_t sK[2][kBKV * kLds];
  __shared__ __attribute__((aligned(16))) bf16_t sV[2][kHd * kLds];
  __shared__ uint8_t sM[2][kBKV];

  // 1D grid.  Non-causal: consecutive workgroups are consecutive query tiles of
  // one head, so the ~1000 resident workgroups stream the same K/V and share
  // it in L2.  Causal: heads vary fastest and query tiles run last-to-first, so
  // the heaviest tiles (which see the most keys) start first.
  const int id = blockIdx.x;
  const int num_bh = static_cast<int>(gridDim.x) / num_qblocks;
  int bh, qb;
  if constexpr (CAUSAL) {
    bh = id % num_bh;
    qb = num_qblocks - 1 - id / num_bh;
  } else {
    qb = id % num_qblocks;
    bh = id / num_qblocks;
  }
  const int b = bh / H;
  const int h = bh - b * H;
  const int q0 = qb * kBQ;
  const int D = H * kHd;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;
  const int qrow = q0 + wave * 32 + l32;  // the query this lane owns

  int kv_limit = S;  // keys >= kv_limit are excluded
  if constexpr (MASK == kMaskPrefix) kv_limit = min(S, static_cast<int>(kv_len[b]));

  bf16_t* ctx_row = ctx + (static_cast<int64_t>(b) * S + qrow) * D + h * kHd;

  if (MASK == kMaskPrefix && q0 >= kv_limit) {
    // Whole query tile is padding: zeros, no work.
    if (qrow < S) {
#pragma unroll
      for (int c = 0; c < 4; ++c)
        *reinterpret_cast<u32x4*>(ctx_row + lhi * 32 + c * 8) = u32x4{0, 0, 0, 0};
    }
    return;
  }

  int kv_end = kv_limit;
  if constexpr (CAUSAL) kv_end = min(kv_end, q0 + kBQ);
  const int nkb = (kv_end + kBKV - 1) / kBKV;

  const int64_t head_off = static_cast<int64_t>(bh) * S * kHd;
  const bf16_t* Qh = Q + head_off;
  const bf16_t* Kh = Kg + head_off;
  const bf16_t* Vh = Vt + static_cast<int64_t>(bh) * kHd * ld_vt;
  const uint8_t* Mh = (MASK == kMaskBytes) ? key_mask + static_cast<int64_t>(b) * S : nullptr;

  // Q fragments (B operand of S^T): lane (q = l32, k-group lhi) holds
  // d = 16*ks + 8*lhi .. +8.
  bf16x8 qf[4];
#pragma unroll
  for (int ks = 0; ks < 4; ++ks) {
    if (qrow < S) {
      qf[ks] = *reinterpret_cast<const bf16x8*>(Qh + static_cast<int64_t>(qrow) * kHd + ks * 16 + lhi * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = static_cast<__bf16>(0.f);
    }
  }

  // Tile loader: K tile = 64 keys x 64 d (512 x 16B chunks), V^T tile = 64 d x
  // 64 keys (512 chunks); 256 threads -> 2 chunks of each per thread.
  u32x4 rk[2], rv[2];
  uint32_t rm = 0;
  auto load_tile = [&](int kb, bool with_v) {
    const int k0 = kb * kBKV;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * kThreads;
      const int row = c >> 3;  // key (K) or d (V^T)
      const int cc = c & 7;    // 16B chunk within the row
      const int key = k0 + row;
      if (key < S) {
        rk[i] = *reinterpret_cast<const u32x4*>(Kh + static_cast<int64_t>(key) * kHd + cc * 8);
      } else {
        rk[i] = u32x4{0, 0, 0, 0};
      }
      if (!with_v) continue;
      const int kv0 = k0 + cc * 8;
      const bf16_t* vp = Vh + static_cast<int64_t>(row) * ld_vt + kv0;
      if (kv0 + 8 <= S) {
        rv[i] = *reinterpret_cast<const u32x4*>(vp);
      } else {
        uint16_t tmp[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) tmp[e] = (kv0 + e < S) ? vp[e] : uint16_t(0);
        rv[i] = u32x4{tmp[0] | (uint32_t(tmp[1]) << 16), tmp[2] | (uint32_t(tmp[3]) << 16),
                      tmp[4] | (uint32_t(tmp[5]) << 16), tmp[6] | (uint32_t(tmp[7]) << 16)};
      }
    }
    if constexpr (MASK == kMaskBytes) {
      if (tid < kBKV) {
        const int key = k0 + tid;
        rm = (key < S) ? Mh[key] : 0;
      }
    }
  };
  auto store_tile = [&](int buf, bool with_v) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(&sK[buf][(c >> 3) * kLds + (c & 7) * 8]) = rk[i];
      if (with_v) *reinterpret_cast<u32x4*>(&sV[buf][(c >> 3) * kLds + (c & 7) * 8]) = rv[i];
    }
    if constexpr (MASK == kMaskBytes) {
      if (tid < kBKV) sM[buf][tid] = static_cast<uint8_t>(rm);
    }
  };

  // Exponent arithmetic: with a power-of-two scale, s = bf16(q.k) * scale is
  // exact, so s - max(s) = (r - max r) * scale with r = bf16(q.k) and
  // exp(s - max) = exp2((r - max r) * (scale * log2 e)), both factors exact.
  // Otherwise s is rounded again after the scale and differences are taken in s.
  const float cexp = POW2_SCALE ? scale * kLog2e : kLog2e;
  auto score_value = [&](float raw) -> float {
    const float r = round_bf16(raw);
    if constexpr (POW2_SCALE) return r;
    else return round_bf16(r * scale);
  };

  // The wavefront's query rows; key tiles with k0 > wq_last are in its future.
  const int wq_first = q0 + wave * 32;
  const int wq_last = wq_first + 31;

  // S^T tile (64 keys x 32 queries) of the current LDS buffer into s[2], already
  // converted to score values, excluded keys set to -inf.
  auto tile_scores = [&](int buf, int k0, f32x16 (&s)[2]) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[0][r] = 0.f;
      s[1][r] = 0.f;
    }
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
        const bf16x8 kf = *reinterpret_cast<const bf16x8*>(
            &sK[buf][(kb32 * 32 + l32) * kLds + ks * 16 + lhi * 8]);
        s[kb32] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb32], 0, 0, 0);
      }
    }
    const bool need_mask = (CAUSAL && k0 + kBKV - 1 > wq_first) || (k0 + kBKV > kv_limit) ||
                           (MASK == kMaskBytes);
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        float v = score_value(s[kb32][r]);
        if (need_mask) {
          const int kl = kb32 * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
          const int key = k0 + kl;
          bool ok = key < kv_limit;
          if constexpr (CAUSAL) ok = ok && key <= qrow;
          if constexpr (MASK == kMaskBytes) ok = ok && sM[buf][kl] != 0;
          v = ok ? v : -INFINITY;
        }
        s[kb32][r] = v;
      }
    }
  };

  // ================= pass 1: row max and row sum of exp(s - max) =================
  // Each lane keeps its own running max/sum over its half of the keys; the two
  // halves (lanes l and l^32) are merged once at the end.
  float m_lane = -INFINITY;
  float l_lane = 0.f;
  if (nkb > 0) {
    load_tile(0, false);
    store_tile(0, false);
  }
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) load_tile(kb + 1, false);
    const int k0 = kb * kBKV;
    if (!CAUSAL || k0 <= wq_last) {
      f32x16 s[2];
      tile_scores(cur, k0, s);
      float mx = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) mx = fmaxf(mx, fmaxf(s[0][r], s[1][r]));
      const float m_new = fmaxf(m_lane, mx);
      const float base = (m_new == -INFINITY) ? 0.f : m_new;
      float acc = l_lane * exp2f((m_lane - base) * cexp);
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        acc += exp2f((s[0][r] - base) * cexp);
        acc += exp2f((s[1][r] - base) * cexp);
      }
      l_lane = acc;
      m_lane = m_new;
    }
    if (kb + 1 < nkb) store_tile(cur ^ 1, false);
    __syncthreads();
  }
  const float m_other = __shfl_xor(m_lane, 32, kWave);
  const float l_other = __shfl_xor(l_lane, 32, kWave);
  const float m_row = fmaxf(m_lane, m_other);
  const float base = (m_row == -INFINITY) ? 0.f : m_row;
  const float l_row = l_lane * exp2f((m_lane - base) * cexp) + l_other * exp2f((m_other - base) * cexp);
  const float inv_l = (l_row > 0.f) ? 1.0f / l_row : 0.f;

  // ========== pass 2: p = bf16(exp(s - max) / sum), context = sum_j p_j v_j ==========
  // P is final when it is rounded (as in the reference), so the PV product
  // accumulates in plain key order with no rescaling.
  f32x16 o[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    o[0][r] = 0.f;
    o[1][r] = 0.f;
  }
  if (nkb > 0) {
    load_tile(0, true);
    store_tile(0, true);
  }
  __syncthreads();
  for (int kb = 0; kb < nkb; ++kb) {
    const int cur = kb & 1;
    if (kb + 1 < nkb) load_tile(kb + 1, true);
    const int k0 = kb * kBKV;
    if (!CAUSAL || k0 <= wq_last) {
      f32x16 s[2];
      tile_scores(cur, k0, s);
      bf16x8 pf[4];
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = exp2f((s[kb32][r] - base) * cexp) * inv_l;
          pf[kb32 * 2 + (r >> 3)][r & 7] = static_cast<__bf16>(p);
        }
      }
#pragma unroll
      for (int db = 0; db < 2; ++db) {
#pragma unroll
        for (int kk = 0; kk < 4; ++kk) {
          const bf16_t* vrow = &sV[cur][(db * 32 + l32) * kLds + 16 * kk + 4 * lhi];
          const u32x2 lo = *reinterpret_cast<const u32x2*>(vrow);
          const u32x2 hi = *reinterpret_cast<const u32x2*>(vrow + 8);
          const u32x4 vv = {lo[0], lo[1], hi[0], hi[1]};
          const bf16x8 vf = __builtin_bit_cast(bf16x8, vv);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[kk], o[db], 0, 0, 0);
        }
      }
    }
    if (kb + 1 < nkb) store_tile(cur ^ 1, true);
    __syncthreads();
  }

  // ---- write context[b, qrow, h*64 + d] = bf16(O) ----
  if (qrow < S) {
    bool zero = !(l_row > 0.f);
    if constexpr (MASK == kMaskPrefix) zero = zero || qrow >= kv_limit;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int d = db * 32 + 8 * i + 4 * lhi;
        u32x2 w = {0u, 0u};
        if (!zero) {
          w = u32x2{pack_bf16x2(o[db][4 * i], o[db][4 * i + 1]),
                    pack_bf16x2(o[db][4 * i + 2], o[db][4 * i + 3])};
        }
        *reinterpret_cast<u32x2*>(ctx_row + d) = w;
      }
    }
  }
}

template <bool CAUSAL, int MASK, bool POW2>
hipError_t launch_attn(const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B,
                       int H, int S, float scale, const int32_t* kv_len, const uint8_t* key_mask,
                       hipStream_t st) {
  const int nqb = (S + kBQ - 1) / kBQ;
  const dim3 grid(static_cast<uint32_t>(B) * H * nqb);
  const int ld_vt = static_cast<int>(vt_stride(S));
  hipLaunchKernelGGL((attn_fwd_hd64_kernel<CAUSAL, MASK, POW2>), grid, dim3(kThreads), 0, st, q,
                     k, vt, ctx, H, S, ld_vt, nqb, scale, kv_len, key_mask);
  return hipGetLastError();
}

template <bool CAUSAL, int MASK>
hipError_t dispatch_pow2(bool pow2, const bf16_t* q, const bf16_t* k, const bf16_t* vt,
                         bf16_t* ctx, int B, int H, int S, float scale, const int32_t* kv_len,
                         const uint8_t* key_mask, hipStream_t st) {
  if (pow2) return launch_attn<CAUSAL, MASK, true>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return launch_attn<CAUSAL, MASK, false>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

template <bool CAUSAL>
hipError_t dispatch_mask(int mask, bool pow2, const bf16_t* q, const bf16_t* k, const bf16_t* vt,
                         bf16_t* ctx, int B, int H, int S, float scale, const int32_t* kv_len,
                         const uint8_t* key_mask, hipStream_t st) {
  if (mask == kMaskPrefix) return dispatch_pow2<CAUSAL, kMaskPrefix>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  if (mask == kMaskBytes) return dispatch_pow2<CAUSAL, kMaskBytes>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return dispatch_pow2<CAUSAL, kMaskNone>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

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

}  // namespace

hipError_t attention_fwd_bf16(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx,
                              int batch, int heads, int seq_len, int head_dim, float scale,
                              bool causal, const int32_t* kv_len, const uint8_t* key_mask,
                              hipStream_t stream) {
  if (head_dim != kHd) return hipErrorInvalidValue;
  if (batch == 0 || seq_len == 0) return hipSuccess;
  int mant_exp = 0;
  const float mant = frexpf(scale, &mant_exp);
  const bool pow2 = (mant == 0.5f);
  const int mask = key_mask != nullptr ? kMaskBytes : (kv_len != nullptr ? kMaskPrefix : kMaskNone);
  if (causal)
    return dispatch_mask<true>(mask, pow2, q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, stream);
  return dispatch_mask<false>(mask, pow2, q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, stream);
}

hipError_t mask_lengths(const uint8_t* mask, int64_t batch, int64_t seq_len, int32_t* kv_len,
                        hipStream_t stream) {
  if (batch == 0) return hipSuccess;
  hipLaunchKernelGGL(mask_lengths_kernel, dim3(static_cast<uint32_t>(batch)), dim3(256), 0, stream,
                     mask, seq_len, kv_len);
  return hipGetLastError();
}

}  // namespace enc
