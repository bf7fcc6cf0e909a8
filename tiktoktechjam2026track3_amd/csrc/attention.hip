// Streaming multi-head attention forward for gfx950, head_dim = 64, bitwise
// equal to the reference's materialised softmax attention.
//
// Scores are never materialised: each workgroup owns BQ = 128 query rows of one
// (batch, head) (32 per wavefront) and streams 64-key tiles of K (and V^T)
// through double-buffered LDS.  Both products put the query on the MFMA N
// dimension (the lane), so every per-query quantity lives in the lane that owns
// the query (lane l: query l%32, key half l/32):
//   S^T[key, q]  = K[key, :] . Q[q, :]        A = K tile (LDS), B = Q (registers)
//   O^T[d, q]   += V^T[d, key] . P^T[key, q]  A = V^T tile (LDS), B = P (registers)
// The K fragment's MFMA row r is fed key perm(r) = 16(i>>1) + 8h + 4(i&1) + j for
// r = 8i + 4h + j, which leaves lane half h holding, for each 16-key group kk,
// keys 16kk + 8h + e (e = 0..7) in consecutive accumulator registers: exactly the
// B operand of the PV MFMA with the reduction index in natural key order, so PV
// accumulates keys in the same order as the reference's matmul(P, V).
//
// Numerics reproduce transformer_benchmark/models.py:55-70 bit for bit:
//   s = bf16(bf16(q.k) * scale)                 (MFMA, fp32 accumulate, rounded)
//   p = bf16(softmax_fp32(s))                   (torch.softmax in fp32, then bf16)
//   context = bf16(sum_j p_j v_j)               (MFMA, fp32 accumulate)
// torch's ROCm softmax computes p differently for the two row-length regimes:
//   rows of <= 2048 keys: e = expf(s - max) (libm-accurate), p = e / sum;
//   longer rows:          e = exp2(rn(s - max) * log2(e)) on the hardware exp
//                         unit, p = e * (1 / sum) with a correctly rounded 1 / sum.
// The softmax sum is accumulated in the order torch's ROCm softmax uses:
//   rows of <= 2048 keys (persistent warp softmax): "lane" lam = key % 64 sums its
//     keys lam, lam+64, ... in order, then a 64-lane butterfly;
//   longer rows (block softmax): "thread" t of 512 sums the 4-key vectors t,
//     t+512, ... in order, then a shuffle-down tree inside each 64-thread warp and
//     a tree over the 8 warp sums.
// Both orders were pinned against torch.softmax on an MI355X by fingerprinting
// the reduction tree.  Because p is rounded after normalisation, the kernel
// sweeps the keys three times: (A) row max, (B) row sum, (C) probabilities + PV.
// In sweep B for long rows, tiles are visited residue-major (tile n = r + 32m,
// r = 0..31) so each 512-thread "thread" partial is completed in key order and
// each warp's 64 partials are live in registers only while that warp is summed.
//
// Tile skipping: with causal masking a workgroup stops at the last key tile its
// last query can see, and a wavefront skips the MFMAs of tiles in its future;
// with prefix padding (kv_len) key tiles past kv_len are never loaded and query
// tiles past kv_len are written as zeros.  Skipped keys contribute exp(-inf) = 0
// in the reference, so skipping them is exact.
#include "common.h"
#include "kernels.h"

namespace enc {

namespace {

constexpr int kHd = 64;
constexpr int kBQ = 128;      // queries per workgroup (32 per wavefront)
constexpr int kBKV = 64;      // keys per tile
constexpr int kLds = 64 + 8;  // padded LDS row (elements)
constexpr int kThreads = 256;
constexpr int kWarpSoftmaxMaxKeys = 2048;  // rows up to this length use the warp order
constexpr float kLog2e = 1.44269504088896340736f;

// exp of (s - max) as the softmax of the given regime computes it.
template <bool BLOCK_ORDER>
__device__ __forceinline__ float softmax_exp(float x) {
  if constexpr (BLOCK_ORDER) {
    return __builtin_amdgcn_exp2f(x * kLog2e);
  } else {
    return expf(x);
  }
}

enum MaskMode : int { kMaskNone = 0, kMaskPrefix = 1, kMaskBytes = 2 };

// key offset inside a 64-key tile held by accumulator register r of block kb32
// in lane half h (see the permutation above)
__device__ __forceinline__ int tile_key(int kb32, int r, int h) {
  const int i = r >> 2, j = r & 3;
  return 32 * kb32 + 16 * (i >> 1) + 8 * h + 4 * (i & 1) + j;
}

template <bool CAUSAL, int MASK, bool POW2_SCALE, bool BLOCK_ORDER>
__global__ void __launch_bounds__(kThreads)
attn_fwd_hd64_kernel(const bf16_t* __restrict__ Q, const bf16_t* __restrict__ Kg,
                     const bf16_t* __restrict__ Vt, bf16_t* __restrict__ ctx, int H, int S,
                     int ld_vt, int num_qblocks, float scale,
                     const int32_t* __restrict__ kv_len, const uint8_t* __restrict__ key_mask) {
  __shared__ __attribute__((aligned(16))) bf16_t sK[2][kBKV * kLds];
  __shared__ __attribute__((aligned(16))) bf16_t sV[2][kHd * kLds];
  __shared__ uint8_t sM[2][kBKV];

  // 1D grid.  Non-causal: consecutive workgroups are consecutive query tiles of
  // one head, so the resident workgroups stream the same K/V and share it in L2.
  // Causal: heads vary fastest and query tiles run last-to-first, so the
  // heaviest tiles (which see the most keys) start first.
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
  // MFMA row l32 of a 32-key block reads K row perm(l32)
  const int krow = 16 * ((l32 >> 3) >> 1) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);

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

  // Runs body(buf, tile) over nkb tiles in the order seq(0), seq(1), ...,
  // double-buffered: the loads of the next tile overlap the current body.
  auto sweep = [&](auto seq, bool with_v, auto body) {
    if (nkb > 0) {
      load_tile(seq(0), with_v);
      store_tile(0, with_v);
    }
    __syncthreads();
    for (int it = 0; it < nkb; ++it) {
      const int cur = it & 1;
      if (it + 1 < nkb) load_tile(seq(it + 1), with_v);
      body(cur, seq(it));
      if (it + 1 < nkb) store_tile(cur ^ 1, with_v);
      __syncthreads();
    }
  };

  const int wq_first = q0 + wave * 32;
  const int wq_last = wq_first + 31;

  // Score tile (64 keys x 32 queries) of LDS buffer `buf` into s[2]: the
  // reference's fp32 view of its bf16 scores, excluded keys = -inf.
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
            &sK[buf][(kb32 * 32 + krow) * kLds + ks * 16 + lhi * 8]);
        s[kb32] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb32], 0, 0, 0);
      }
    }
    const bool need_mask = (CAUSAL && k0 + kBKV - 1 > wq_first) || (k0 + kBKV > kv_limit) ||
                           (MASK == kMaskBytes);
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float rq = round_bf16(s[kb32][r]);
        float v = POW2_SCALE ? rq * scale : round_bf16(rq * scale);
        if (need_mask) {
          const int kl = tile_key(kb32, r, lhi);
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
  auto natural = [](int it) { return it; };

  // ============================ sweep A: row max ============================
  float m_lane = -INFINITY;
  sweep(natural, false, [&](int buf, int kb) {
    const int k0 = kb * kBKV;
    if (CAUSAL && k0 > wq_last) return;
    f32x16 s[2];
    tile_scores(buf, k0, s);
#pragma unroll
    for (int r = 0; r < 16; ++r) m_lane = fmaxf(m_lane, fmaxf(s[0][r], s[1][r]));
  });
  const float row_max = fmaxf(m_lane, __shfl_xor(m_lane, 32, kWave));

  // ======================= sweep B: row sum of expf(s - max) =======================
  float row_sum;
  if constexpr (!BLOCK_ORDER) {
    // warp order: partial[lam] over keys lam, lam+64, ... (lam = key % 64)
    float part[2][16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      part[0][r] = 0.f;
      part[1][r] = 0.f;
    }
    sweep(natural, false, [&](int buf, int kb) {
      const int k0 = kb * kBKV;
      if (CAUSAL && k0 > wq_last) return;
      f32x16 s[2];
      tile_scores(buf, k0, s);
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int r = 0; r < 16; ++r) part[kb32][r] += softmax_exp<false>(s[kb32][r] - row_max);
    });
    // 64-lane butterfly; lam bits: 5 = kb32, 4 = i>>1 (reg bit 3), 3 = lane half,
    // 2 = i&1 (reg bit 2), 1..0 = j (reg bits 1..0)
    float a[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) a[r] = part[0][r] + part[1][r];             // offset 32
    float c[8];
#pragma unroll
    for (int r = 0; r < 8; ++r) c[r] = a[r] + a[r + 8];                      // offset 16
#pragma unroll
    for (int r = 0; r < 8; ++r) c[r] = c[r] + __shfl_xor(c[r], 32, kWave);  // offset 8
    float d4[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) d4[r] = c[r] + c[r + 4];                     // offset 4
    const float e2a = d4[0] + d4[2], e2b = d4[1] + d4[3];                    // offset 2
    row_sum = e2a + e2b;                                                     // offset 1
  } else {
    // block order: "thread" t (of 512) sums 4-key vectors t, t+512, ...; tile
    // n = r + 32 m holds the vectors of threads 16 r .. 16 r + 15.  Tiles are
    // visited residue-major; "warp" w covers residues 4w .. 4w+3.
    auto resmajor = [&](int it) {
      int r = 0;
      int acc = 0;
      while (true) {
        const int cnt = (nkb - r + 31) / 32;  // tiles with residue r
        if (it < acc + cnt) return r + 32 * (it - acc);
        acc += cnt;
        ++r;
      }
    };
    float warp_sum[8];
    float part[4][8];  // [residue within warp][vector slot 4*kb32 + i]
#pragma unroll
    for (int w = 0; w < 8; ++w) warp_sum[w] = 0.f;
#pragma unroll
    for (int q = 0; q < 4; ++q)
#pragma unroll
      for (int v = 0; v < 8; ++v) part[q][v] = 0.f;
    int cur_warp = 0;
    auto flush_warp = [&](int w) {
      // shuffle-down tree over lam = 16 rr + u, u = 8 kb32 + 4 (i>>1) + 2 h + (i&1):
      // offsets 32, 16 (rr), 8 (kb32), 4 (i>>1), 2 (lane half), 1 (i&1)
      float t8[8];
#pragma unroll
      for (int v = 0; v < 8; ++v) t8[v] = (part[0][v] + part[2][v]) + (part[1][v] + part[3][v]);
      float t4[4];
#pragma unroll
      for (int v = 0; v < 4; ++v) t4[v] = t8[v] + t8[v + 4];                   // offset 8 (kb32)
      float t2[2];
#pragma unroll
      for (int v = 0; v < 2; ++v) t2[v] = t4[v] + t4[v + 2];                   // offset 4 (i>>1)
#pragma unroll
      for (int v = 0; v < 2; ++v) t2[v] = t2[v] + __shfl_xor(t2[v], 32, kWave);  // offset 2
      const float ws = t2[0] + t2[1];                                          // offset 1 (i&1)
#pragma unroll
      for (int ww = 0; ww < 8; ++ww)
        if (ww == w) warp_sum[ww] = ws;
#pragma unroll
      for (int q = 0; q < 4; ++q)
#pragma unroll
        for (int v = 0; v < 8; ++v) part[q][v] = 0.f;
    };
    sweep(resmajor, false, [&](int buf, int kb) {
      const int k0 = kb * kBKV;
      const int r = kb & 31;
      const int w = r >> 2;
      while (cur_warp < w) {  // warps whose residues are complete are reduced
        flush_warp(cur_warp);
        ++cur_warp;
      }
      if (CAUSAL && k0 > wq_last) return;
      f32x16 s[2];
      tile_scores(buf, k0, s);
      const int rr = r & 3;
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float acc = 0.f;
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (q == rr) acc = part[q][4 * kb32 + i];
#pragma unroll
          for (int j = 0; j < 4; ++j) acc += softmax_exp<true>(s[kb32][4 * i + j] - row_max);
#pragma unroll
          for (int q = 0; q < 4; ++q)
            if (q == rr) part[q][4 * kb32 + i] = acc;
        }
      }
    });
    while (cur_warp < 8) {
      flush_warp(cur_warp);
      ++cur_warp;
    }
    // tree over the 8 warp sums (offsets 4, 2, 1)
    const float a0 = warp_sum[0] + warp_sum[4], a1 = warp_sum[1] + warp_sum[5];
    const float a2 = warp_sum[2] + warp_sum[6], a3 = warp_sum[3] + warp_sum[7];
    row_sum = (a0 + a2) + (a1 + a3);
  }

  // ================== sweep C: p = bf16(softmax), context += P V ==================
  const float inv_sum = 1.0f / row_sum;  // block-order epilogue multiplies by it
  f32x16 o[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    o[0][r] = 0.f;
    o[1][r] = 0.f;
  }
  sweep(natural, true, [&](int buf, int kb) {
    const int k0 = kb * kBKV;
    if (CAUSAL && k0 > wq_last) return;
    f32x16 s[2];
    tile_scores(buf, k0, s);
    bf16x8 pf[4];
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = softmax_exp<BLOCK_ORDER>(s[kb32][r] - row_max);
        const float p = BLOCK_ORDER ? e * inv_sum : e / row_sum;
        pf[kb32 * 2 + (r >> 3)][r & 7] = static_cast<__bf16>(p);
      }
    }
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(
            &sV[buf][(db * 32 + l32) * kLds + 16 * kk + 8 * lhi]);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[kk], o[db], 0, 0, 0);
      }
    }
  });

  // ---- write context[b, qrow, h*64 + d] = bf16(O) ----
  if (qrow < S) {
    bool zero = !(row_sum > 0.f);
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

template <bool CAUSAL, int MASK, bool POW2, bool BLOCK_ORDER>
hipError_t launch_attn(const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B,
                       int H, int S, float scale, const int32_t* kv_len, const uint8_t* key_mask,
                       hipStream_t st) {
  const int nqb = (S + kBQ - 1) / kBQ;
  const dim3 grid(static_cast<uint32_t>(B) * H * nqb);
  const int ld_vt = static_cast<int>(vt_stride(S));
  hipLaunchKernelGGL((attn_fwd_hd64_kernel<CAUSAL, MASK, POW2, BLOCK_ORDER>), grid, dim3(kThreads),
                     0, st, q, k, vt, ctx, H, S, ld_vt, nqb, scale, kv_len, key_mask);
  return hipGetLastError();
}

template <bool CAUSAL, int MASK, bool POW2>
hipError_t dispatch_order(const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B,
                          int H, int S, float scale, const int32_t* kv_len,
                          const uint8_t* key_mask, hipStream_t st) {
  if (S > kWarpSoftmaxMaxKeys)
    return launch_attn<CAUSAL, MASK, POW2, true>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return launch_attn<CAUSAL, MASK, POW2, false>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

template <bool CAUSAL, int MASK>
hipError_t dispatch_pow2(bool pow2, const bf16_t* q, const bf16_t* k, const bf16_t* vt,
                         bf16_t* ctx, int B, int H, int S, float scale, const int32_t* kv_len,
                         const uint8_t* key_mask, hipStream_t st) {
  if (pow2) return dispatch_order<CAUSAL, MASK, true>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return dispatch_order<CAUSAL, MASK, false>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
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

bool attention_seq_supported(int64_t seq_len) {
  // torch's long-row softmax folds 4-element vectors; other lengths are not pinned
  return seq_len <= kWarpSoftmaxMaxKeys || seq_len % 4 == 0;
}

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
