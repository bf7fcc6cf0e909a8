// Streaming (online-softmax) multi-head attention forward for gfx950,
// head_dim = 64.  Scores are never materialised and every key is visited once.
//
// Work decomposition: a workgroup of NW wavefronts owns NW * 32 query rows of
// one (batch, head); wavefront w owns 32 of them.  64-key tiles of K and V^T
// stream through a two-stage LDS ring filled with direct global->LDS loads
// (global_load_lds_dwordx4), so K/V bytes never pass through VGPRs.  Both
// products put the query on the MFMA N dimension (the lane):
//   S^T[key, q] = K[key, :] . Q[q, :]        A = K tile (LDS), B = Q (registers)
//   O^T[d, q]  += V^T[d, key] . P^T[key, q]  A = V^T tile (LDS), B = P (registers)
// The K fragment's MFMA row r is fed key perm(r) = 16(i>>1) + 8h + 4(i&1) + j
// for r = 8i + 4h + j, so lane half h ends up holding, for every 16-key group,
// keys 16kk + 8h + e (e = 0..7) in consecutive accumulator registers: exactly
// the B operand of the PV MFMA.  P therefore goes from the score accumulators
// to the PV MFMA without an LDS round trip, and every per-query quantity (row
// max, row sum, rescale factor) lives in the lane that owns the query.
//
// Numerics follow transformer_benchmark/models.py:55-70 at its rounding points:
//   s = bf16(bf16(q.k) * scale)            (MFMA, fp32 accumulate, rounded)
//   p = exp(s - m) in fp32, rounded to bf16 for the PV MFMA (fp32 accumulate)
//   context = bf16(sum_j p_j v_j / sum_j p_j)
// The reference normalises p before its bf16 rounding (softmax then .to(bf16));
// here the unnormalised exponentials are rounded and the fp32 sum divides the
// fp32 context once at the end.  Both round each probability once to bf16, so
// the two contexts differ by bf16 rounding noise of the weights, well inside
// the bf16 tolerance the build is held to.  (The exact three-sweep kernel in
// attention.hip reproduces the reference bit for bit when that is needed.)
//
// Online softmax with lazy rescaling: the running max m of a query is only
// raised when a tile's max exceeds it by more than 2^8 in the exponential, so
// almost every tile skips the O *= alpha rescale; unnormalised weights stay
// below 2^8, far inside fp32 and bf16 range.
//
// Tile skipping: with causal masking a workgroup stops at the last key tile its
// last query can see and a wavefront skips tiles entirely in its future; with
// prefix padding (kv_len) key tiles at or past kv_len are never loaded and
// query tiles past kv_len are written as zeros.  Skipped keys contribute
// exp(-inf) = 0 in the reference, so skipping them is exact.
#include "common.h"
#include "kernels.h"

namespace enc {

namespace {

constexpr int kHd = 64;
constexpr int kBKV = 64;                      // keys per tile
constexpr int kTileElems = kBKV * kHd;        // one K or V^T tile, bf16 elements
constexpr float kLog2e = 1.44269504088896340736f;
constexpr float kLazyRescaleLog2 = 8.0f;      // rescale when the max grows by > 2^8

enum MaskMode : int { kMaskNone = 0, kMaskPrefix = 1, kMaskBytes = 2 };

// LDS tile = 64 rows (keys of K, head channels of V^T) x 8 chunks of 16 bytes.
// Chunk c of row r sits in slot c ^ (r & 7), so the 32 rows one MFMA fragment
// read touches at a fixed chunk fall in distinct bank groups.
__device__ __forceinline__ int tile_off(int row, int chunk) { return row * kHd + ((chunk ^ (row & 7)) << 3); }

// s_waitcnt immediate: wait until no vector-memory operation is outstanding
// (expcnt and lgkmcnt left at their no-wait maxima; gfx9 encoding).
constexpr int kWaitVm0 = (7 << 4) | (15 << 8);

// key offset inside a 64-key tile held by accumulator register r of 32-key
// block kb32 in lane half h
__device__ __forceinline__ int tile_key(int kb32, int r, int h) {
  const int i = r >> 2, j = r & 3;
  return 32 * kb32 + 16 * (i >> 1) + 8 * h + 4 * (i & 1) + j;
}

template <int NW, bool CAUSAL, int MASK, bool POW2_SCALE>
__global__ void __launch_bounds__(NW * kWave)
flash_attn_hd64_kernel(const bf16_t* __restrict__ Q, const bf16_t* __restrict__ Kg,
                       const bf16_t* __restrict__ Vt, bf16_t* __restrict__ ctx, int H, int S,
                       int ld_vt, int num_qblocks, float scale,
                       const int32_t* __restrict__ kv_len, const uint8_t* __restrict__ key_mask) {
  constexpr int kThreads = NW * kWave;
  constexpr int kBQ = NW * 32;
  __shared__ __attribute__((aligned(16))) bf16_t sK[2][kTileElems];
  __shared__ __attribute__((aligned(16))) bf16_t sV[2][kTileElems];
  __shared__ uint8_t sM[2][kBKV];

  // Block -> (batch*head, query tile).  Non-causal: MI355X hands consecutive
  // workgroups to its 8 XCDs round-robin; the id is remapped so each XCD walks
  // a contiguous run of query tiles of one head, whose K/V then stream once
  // through that XCD's L2.  Causal: heads vary fastest and query tiles run
  // last-to-first, so the heaviest tiles (most keys) start first.
  const int nblocks = static_cast<int>(gridDim.x);
  const int num_bh = nblocks / num_qblocks;
  int bh, qb;
  if constexpr (CAUSAL) {
    const int id = blockIdx.x;
    bh = id % num_bh;
    qb = num_qblocks - 1 - id / num_bh;
  } else {
    const int pid = blockIdx.x;
    const int xcd = pid % 8, slot = pid / 8;
    const int base = nblocks / 8, rem = nblocks % 8;
    const int id = xcd * base + min(xcd, rem) + slot;
    qb = id % num_qblocks;
    bh = id / num_qblocks;
  }
  const int b = bh / H;
  const int h = bh - b * H;
  const int q0 = qb * kBQ;
  const int D = H * kHd;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  // wavefront index as a scalar, so per-tile decisions stay uniform branches
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int l32 = lane & 31;
  const int lhi = lane >> 5;
  const int qrow = q0 + wave * 32 + l32;  // the query this lane owns

  int kv_limit = S;  // keys >= kv_limit are excluded
  if constexpr (MASK == kMaskPrefix) kv_limit = min(S, static_cast<int>(kv_len[b]));

  bf16_t* ctx_row = ctx + (static_cast<int64_t>(b) * S + qrow) * D + h * kHd;
  if (MASK == kMaskPrefix && q0 >= kv_limit) {
    // whole query tile is padding: zeros, no work
    if (qrow < S) {
#pragma unroll
      for (int c = 0; c < 4; ++c) *reinterpret_cast<u32x4*>(ctx_row + lhi * 32 + c * 8) = u32x4{0, 0, 0, 0};
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
  // channels 16*ks + 8*lhi .. +8.
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

  // ---- tile loads ----
  // Full tiles: load instruction j of wavefront w fills LDS rows 8(NW j + w) ..
  // +7 (64 lanes x 16 bytes, consecutive); lane L writes row 8(NW j + w) + L/8,
  // slot L%8, which holds chunk (L%8) ^ (L/8) of that row.
  const int ld_row = lane >> 3;
  const int ld_chunk = (lane & 7) ^ ld_row;
  auto issue_full = [&](int buf, int k0) {
#pragma unroll
    for (int j = 0; j < 8 / NW; ++j) {
      const int row0 = 8 * (NW * j + wave);
      const int row = row0 + ld_row;
      __builtin_amdgcn_global_load_lds(Kh + static_cast<int64_t>(k0 + row) * kHd + ld_chunk * 8,
                                       &sK[buf][row0 * kHd], 16, 0, 0);
      __builtin_amdgcn_global_load_lds(Vh + static_cast<int64_t>(row) * ld_vt + k0 + ld_chunk * 8,
                                       &sV[buf][row0 * kHd], 16, 0, 0);
    }
  };
  // The tile that crosses seq_len goes through registers: keys >= S read as
  // zeros (V^T's padding columns are never read, so they may hold anything).
  auto load_edge = [&](int buf, int k0) {
    for (int c = tid; c < kBKV * 8; c += kThreads) {
      const int row = c >> 3, chunk = c & 7;
      u32x4 kv = u32x4{0, 0, 0, 0};
      if (k0 + row < S) kv = *reinterpret_cast<const u32x4*>(Kh + static_cast<int64_t>(k0 + row) * kHd + chunk * 8);
      *reinterpret_cast<u32x4*>(&sK[buf][tile_off(row, chunk)]) = kv;
      const int key = k0 + chunk * 8;
      const bf16_t* vp = Vh + static_cast<int64_t>(row) * ld_vt + key;
      uint16_t t[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = (key + e < S) ? vp[e] : uint16_t(0);
      *reinterpret_cast<u32x4*>(&sV[buf][tile_off(row, chunk)]) =
          u32x4{t[0] | (uint32_t(t[1]) << 16), t[2] | (uint32_t(t[3]) << 16),
                t[4] | (uint32_t(t[5]) << 16), t[6] | (uint32_t(t[7]) << 16)};
    }
  };
  auto issue_tile = [&](int buf, int kb) {
    const int k0 = kb * kBKV;
    if (k0 + kBKV <= S) {
      issue_full(buf, k0);
    } else {
      load_edge(buf, k0);
    }
    if constexpr (MASK == kMaskBytes) {
      if (tid < kBKV) sM[buf][tid] = (k0 + tid < S) ? Mh[k0 + tid] : uint8_t(0);
    }
  };

  const int wq_first = q0 + wave * 32;
  const int wq_last = wq_first + 31;
  // exp2 of (s - m) * log2(e): with a power-of-two scale the scaled score is
  // exact, so the scale folds into the exp2 multiplier.
  const float c_exp = POW2_SCALE ? scale * kLog2e : kLog2e;

  float m_run = -INFINITY;  // running max (unscaled units when POW2_SCALE)
  float l_run = 0.f;        // this lane half's share of the running sum
  f32x16 o[2];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    o[0][r] = 0.f;
    o[1][r] = 0.f;
  }

  if (nkb > 0) issue_tile(0, 0);
  __builtin_amdgcn_s_waitcnt(kWaitVm0);
  __syncthreads();

  for (int it = 0; it < nkb; ++it) {
    const int buf = it & 1;
    if (it + 1 < nkb) issue_tile(buf ^ 1, it + 1);
    const int k0 = it * kBKV;
    if (!(CAUSAL && k0 > wq_last)) {
      // ---- S^T = K . Q^T for the 64-key tile ----
      f32x16 s[2];
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[0][r] = 0.f;
        s[1][r] = 0.f;
      }
#pragma unroll
      for (int ks = 0; ks < 4; ++ks) {
#pragma unroll
        for (int kb32 = 0; kb32 < 2; ++kb32) {
          const bf16x8 kf =
              *reinterpret_cast<const bf16x8*>(&sK[buf][tile_off(kb32 * 32 + krow, 2 * ks + lhi)]);
          s[kb32] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb32], 0, 0, 0);
        }
      }
      // ---- round to the reference's bf16 scores, mask, tile max ----
      const bool need_mask = (CAUSAL && k0 + kBKV - 1 > wq_first) || (k0 + kBKV > kv_limit) ||
                             (MASK == kMaskBytes);
      float mt = -INFINITY;
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          float v = round_bf16(s[kb32][r]);
          if constexpr (!POW2_SCALE) v = round_bf16(v * scale);
          if (need_mask) {
            const int kl = tile_key(kb32, r, lhi);
            const int key = k0 + kl;
            bool ok = key < kv_limit;
            if constexpr (CAUSAL) ok = ok && key <= qrow;
            if constexpr (MASK == kMaskBytes) ok = ok && sM[buf][kl] != 0;
            v = ok ? v : -INFINITY;
          }
          s[kb32][r] = v;
          mt = fmaxf(mt, v);
        }
      }
      mt = fmaxf(mt, __shfl_xor(mt, 32, kWave));
      // ---- lazy rescale: only when the max grows by more than 2^8 ----
      const bool grow = (mt - m_run) * c_exp > kLazyRescaleLog2;  // false for NaN (both -inf)
      if (__builtin_amdgcn_ballot_w64(grow) != 0) {
        const float m_new = fmaxf(m_run, mt);
        const float alpha = (m_run == -INFINITY) ? 0.f : __builtin_amdgcn_exp2f((m_run - m_new) * c_exp);
        m_run = m_new;
        l_run *= alpha;
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          o[0][r] *= alpha;
          o[1][r] *= alpha;
        }
      }
      const float m_off = (m_run == -INFINITY) ? 0.f : m_run * c_exp;
      // ---- p = exp(s - m) -> bf16 B operand of the PV product ----
      bf16x8 pf[4];
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float p = __builtin_amdgcn_exp2f(fmaf(s[kb32][r], c_exp, -m_off));
          l_run += p;
          pf[kb32 * 2 + (r >> 3)][r & 7] = static_cast<__bf16>(p);
        }
      }
      // ---- O^T += V^T . P^T ----
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
        for (int db = 0; db < 2; ++db) {
          const bf16x8 vf =
              *reinterpret_cast<const bf16x8*>(&sV[buf][tile_off(db * 32 + l32, 2 * kk + lhi)]);
          o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[kk], o[db], 0, 0, 0);
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
  }

  // ---- context[b, qrow, h*64 + d] = bf16(O / l) ----
  const float l_tot = l_run + __shfl_xor(l_run, 32, kWave);
  if (qrow < S) {
    bool zero = !(l_tot > 0.f);
    if constexpr (MASK == kMaskPrefix) zero = zero || qrow >= kv_limit;
    const float inv = zero ? 0.f : 1.0f / l_tot;
#pragma unroll
    for (int db = 0; db < 2; ++db) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = db * 32 + 8 * g + 4 * lhi;
        u32x2 w = {0u, 0u};
        if (!zero) {
          w = u32x2{pack_bf16x2(o[db][4 * g] * inv, o[db][4 * g + 1] * inv),
                    pack_bf16x2(o[db][4 * g + 2] * inv, o[db][4 * g + 3] * inv)};
        }
        *reinterpret_cast<u32x2*>(ctx_row + d) = w;
      }
    }
  }
}

template <int NW, bool CAUSAL, int MASK, bool POW2>
hipError_t launch_flash(const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B, int H,
                        int S, float scale, const int32_t* kv_len, const uint8_t* key_mask,
                        hipStream_t st) {
  constexpr int kBQ = NW * 32;
  const int nqb = (S + kBQ - 1) / kBQ;
  const dim3 grid(static_cast<uint32_t>(B) * H * nqb);
  const int ld_vt = static_cast<int>(vt_stride(S));
  hipLaunchKernelGGL((flash_attn_hd64_kernel<NW, CAUSAL, MASK, POW2>), grid, dim3(NW * kWave), 0, st, q, k,
                     vt, ctx, H, S, ld_vt, nqb, scale, kv_len, key_mask);
  return hipGetLastError();
}

template <bool CAUSAL, int MASK, bool POW2>
hipError_t pick_waves(const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B, int H, int S,
                      float scale, const int32_t* kv_len, const uint8_t* key_mask, hipStream_t st) {
  // Small problems use one-wavefront workgroups (32 queries) so more of the
  // 256 CUs get work; larger ones share each K/V tile among 4 wavefronts.
  const int64_t groups128 = static_cast<int64_t>(B) * H * ((S + 127) / 128);
  if (groups128 < 512)
    return launch_flash<1, CAUSAL, MASK, POW2>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return launch_flash<4, CAUSAL, MASK, POW2>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

template <bool CAUSAL, int MASK>
hipError_t pick_scale(bool pow2, const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B, int H,
                      int S, float scale, const int32_t* kv_len, const uint8_t* key_mask, hipStream_t st) {
  if (pow2) return pick_waves<CAUSAL, MASK, true>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return pick_waves<CAUSAL, MASK, false>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

template <bool CAUSAL>
hipError_t pick_mask(int mask, bool pow2, const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx,
                     int B, int H, int S, float scale, const int32_t* kv_len, const uint8_t* key_mask,
                     hipStream_t st) {
  if (mask == kMaskPrefix)
    return pick_scale<CAUSAL, kMaskPrefix>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  if (mask == kMaskBytes)
    return pick_scale<CAUSAL, kMaskBytes>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return pick_scale<CAUSAL, kMaskNone>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

}  // namespace

hipError_t flash_attention_fwd_bf16(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx,
                                    int batch, int heads, int seq_len, int head_dim, float scale,
                                    bool causal, const int32_t* kv_len, const uint8_t* key_mask,
                                    hipStream_t stream) {
  if (head_dim != kHd) return hipErrorInvalidValue;
  if (batch == 0 || seq_len == 0) return hipSuccess;
  int mant_exp = 0;
  const bool pow2 = frexpf(scale, &mant_exp) == 0.5f;
  const int mask = key_mask != nullptr ? kMaskBytes : (kv_len != nullptr ? kMaskPrefix : kMaskNone);
  if (causal) return pick_mask<true>(mask, pow2, q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, stream);
  return pick_mask<false>(mask, pow2, q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask, stream);
}

}  // namespace enc
