// Streaming multi-head attention forward for gfx950, head_dim 8, 32, 64, 128
// or 256, bitwise
// equal to the reference's materialised softmax attention.
//
// Scores are never materialised: each workgroup owns BQ = NW * 32 query rows
// of one (batch, head) (32 per wavefront) and streams 64-key tiles of K (and
// V^T) through a two-stage LDS ring filled with direct buffer->LDS loads
// (buffer_load_dwordx4 ... lds).  Both products put the query on the MFMA N
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
//   rows of <= 2048 keys: e = expf(s - max) (device-library expf), p = e / sum;
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
//
// Cost notes.  The kernel is bound by VALU work per score, not by the MFMAs:
//   * sweep A takes the max of the raw fp32 dot products and rounds it once at
//     the end; rounding to bf16 (and scaling by a positive scale) is monotonic,
//     so max(bf16(x)) = bf16(max(x));
//   * the division of the short-row regime, p = RN(e / sum), is evaluated as
//     q0 = RN(e * r), rem = fma(-q0, sum, e), p = fma(rem, r, q0) with
//     r = RN(1 / sum): Markstein's correction step, which gives the correctly
//     rounded quotient whenever no intermediate underflows.  Rows whose
//     smallest weight could underflow (min s - max < -69, e < 2^-100) use the
//     IEEE division instead (one branch per wavefront).
// In sweep B for long rows, tiles are visited residue-major (tile n = r + 32m,
// r = 0..31) so each 512-thread "thread" partial is completed in key order and
// each warp's 64 partials are live in registers only while that warp is summed.
//
// Tile skipping: with causal masking a workgroup stops at the last key tile its
// last query can see, and a wavefront skips the MFMAs of tiles in its future;
// with prefix padding (kv_len) key tiles past kv_len are never loaded and query
// tiles past kv_len are written as zeros.  Skipped keys contribute exp(-inf) = 0
// in the reference, and adding 0 leaves a partial sum unchanged, so skipping
// them is exact.
#pragma once

#include <type_traits>

#include "common.h"
#include "kernels.h"

namespace enc {

namespace {

constexpr int kBKV = 64;                   // keys per tile
constexpr int kWarpSoftmaxMaxKeys = 2048;  // rows up to this length use the warp order
constexpr float kLog2e = 1.44269504088896340736f;
// below this weight (s - max < -69.3) the Markstein quotient is not used
constexpr float kMinFastGap = -69.0f;

enum MaskMode : int { kMaskNone = 0, kMaskPrefix = 1, kMaskBytes = 2 };

// LDS tiles, in 16-byte chunks of 8 bf16:
//   K tile:   64 keys x HD channels, HD / 8 chunks per row;
//   V^T tile: HD channels x 64 keys, 8 chunks per row.
// Chunk c of row r sits in slot c ^ swz(r), so the rows one MFMA fragment
// read touches at a fixed chunk spread over distinct bank groups.  A 16-byte
// read serves 16 lanes per LDS cycle, here 16 consecutive rows (in K's
// permuted row order, still rows 16k .. 16k+15); with 128-byte rows (8
// chunks: K at head dim 64, every V^T tile) the row's parity picks the bank
// half and swz(r) = (r >> 1) & 7 the 16-byte group inside it, so those 16
// rows hit 16 distinct groups (r & 7 would pair rows r and r + 8).  Other
// head dims keep c ^ (r & m), m = min(chunks per row, 8) - 1.
template <int HD>
__device__ __forceinline__ int k_swz(int row) {
  constexpr int kSwz = (HD / 8 < 8 ? HD / 8 : 8) - 1;
  if constexpr (HD == 64) {
    return (row >> 1) & 7;
  } else {
    return row & kSwz;
  }
}
template <int HD>
__device__ __forceinline__ int k_off(int row, int chunk) {
  return row * HD + ((chunk ^ k_swz<HD>(row)) << 3);
}
__device__ __forceinline__ int v_swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int v_off(int row, int chunk) { return row * kBKV + ((chunk ^ v_swz(row)) << 3); }

// s_waitcnt immediate: wait until no vector-memory operation is outstanding
// (expcnt and lgkmcnt left at their no-wait maxima; gfx9 encoding).
constexpr int kWaitVm0 = (7 << 4) | (15 << 8);

// key offset inside a 64-key tile held by accumulator register r of block kb32
// in lane half h (see the permutation above)
__device__ __forceinline__ int tile_key(int kb32, int r, int h) {
  const int i = r >> 2, j = r & 3;
  return 32 * kb32 + 16 * (i >> 1) + 8 * h + 4 * (i & 1) + j;
}

// RES > 0: short rows (at most RES tiles): every K/V tile is loaded into LDS
// once and the three sweeps read them from there, with no further loads or
// barriers.  RES == 0: the two-stage ring streams the tiles for each sweep.
// NW == 2 with RES == 2 (key split): the two wavefronts share one block of 32
// queries, wavefront t taking key tile t through the max, exponential and
// probability work (the per-score VALU work, which bounds these short rows);
// the exchanges keep the reference's order: every per-key partial sum is
// e(tile 0) + e(tile 1), and wavefront 0 runs the one P.V MFMA chain over
// both tiles, with wavefront 1's probabilities.
// OCC is the wavefronts per SIMD the register allocation must allow (1: no
// bound).  Long head-dim-64 rows with at least four workgroups per CU use 4
// (at most 128 VGPRs, a few spilled; see dispatch_order); most head-dim-64
// short rows use 3 with the half-tile sweeps (kHalfTiles: at most 168
// VGPRs, see dispatch_order).
template <int HD, int NW, bool CAUSAL, int MASK, bool POW2_SCALE, bool BLOCK_ORDER, int RES, int OCC>
__global__ void __launch_bounds__(NW * kWave, OCC)
attn_fwd_kernel(const bf16_t* __restrict__ Q, const bf16_t* __restrict__ Kg,
                     const bf16_t* __restrict__ Vt, bf16_t* __restrict__ ctx, int H, int S,
                     int ld_vt, int num_qblocks, float scale,
                     const int32_t* __restrict__ kv_len, const uint8_t* __restrict__ key_mask) {
  static_assert(HD == 8 || HD == 32 || HD == 64 || HD == 128 || HD == 256, "head_dim 8, 32, 64, 128 or 256");
  constexpr bool kSplit = NW == 2 && RES == 2;
  static_assert(NW != 2 || (RES == 2 && !BLOCK_ORDER), "two wavefronts: key split of two resident tiles");
  // short-row regime with a power-of-two scale: gaps stay unscaled, the scale
  // folds into expf's constants (exp_gap below)
  constexpr bool kFoldScale = POW2_SCALE && !BLOCK_ORDER;
  // Short rows streamed through the ring at three wavefronts per SIMD: sweeps
  // B and C work on one 32-key half of a tile at a time, so that half of the
  // scores, weights and P fragments are live at once (at most 168 VGPRs
  // instead of 250, none spilled).  Same MFMA chains and per-score operations
  // in the same order, so the same bits.
  constexpr bool kHalfTiles = !BLOCK_ORDER && RES == 0 && OCC == 3;
  constexpr int kThreads = NW * kWave;
  constexpr int kBQ = kSplit ? 32 : NW * 32;
  constexpr int kTileElems = kBKV * HD;  // one K or V^T tile, bf16 elements
  constexpr int kChunksK = HD / 8;       // 16-byte chunks per K row
  // 16-deep MFMA steps of q.k.  Head dim 8 runs one step whose upper 8
  // reduction lanes (lane half 1) hold zeros in both operands.
  constexpr int kKSteps = HD < 16 ? 1 : HD / 16;
  // 32-channel blocks of the context.  Head dim 8 uses MFMA rows 0..7 of one
  // block; the other rows read V^T rows modulo 8 and are never written.
  constexpr int kDBlocks = HD < 32 ? 1 : HD / 32;
  constexpr int kSlabs = HD / 8;  // 1 KiB load instructions per K (or V^T) tile
  // K, V^T and key-mask tiles live in dynamic LDS sized at launch
  // (attn_lds_bytes): a static __shared__ array whose size depends on a
  // template parameter loses the kernel's host launch stub in this compiler.
  constexpr int kBufs = RES > 0 ? RES : 2;
  // (flat pointers: a pointer-to-array type whose bound depends on HD also
  // loses the host launch stub)
  extern __shared__ __attribute__((aligned(16))) bf16_t attn_lds[];
  bf16_t* sK = attn_lds;                        // buffer t at sK + t * kTileElems
  bf16_t* sV = attn_lds + kBufs * kTileElems;   // buffer t at sV + t * kTileElems
  uint8_t (*sM)[kBKV] = reinterpret_cast<uint8_t (*)[kBKV]>(attn_lds + 2 * kBufs * kTileElems);
  // key split exchange areas (after the tiles, 16-byte aligned): the row max
  // and min per wavefront and lane, then the weights e of each wavefront's
  // tile ([wavefront][32 registers][64 lanes]), then wavefront 1's bf16
  // probabilities ([64 lanes][4 fragments])
  float* x_mm = reinterpret_cast<float*>(attn_lds) + (2 * kBufs * kTileElems * 2 + kBufs * kBKV + 15) / 16 * 4;
  float* x_e = x_mm + 2 * 2 * kWave;
  bf16x8* x_p = reinterpret_cast<bf16x8*>(x_e + 2 * 32 * kWave);

  // Block -> (batch*head, query tile).  Non-causal: MI355X hands consecutive
  // workgroups to its 8 XCDs round-robin; the id is remapped so each XCD walks
  // a contiguous run of query tiles of one head, whose K/V then stream through
  // that XCD's L2 once for all of them.  Causal: heads vary fastest and query
  // tiles run last-to-first, so the heaviest tiles (most keys) start first.
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
  const int D = H * HD;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  // wavefront index as a scalar, so per-tile decisions stay uniform branches
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int l32 = lane & 31;
  const int lhi = lane >> 5;
  const int qrow = q0 + (kSplit ? 0 : wave * 32) + l32;  // the query this lane owns

  int kv_limit = S;  // keys >= kv_limit are excluded
  if constexpr (MASK == kMaskPrefix) kv_limit = min(S, static_cast<int>(kv_len[b]));

  bf16_t* ctx_row = ctx + (static_cast<int64_t>(b) * S + qrow) * D + h * HD;

  if (MASK == kMaskPrefix && q0 >= kv_limit) {
    // Whole query tile is padding: zeros, no work.
    if (qrow < S && (!kSplit || wave == 0)) {
      if constexpr (HD >= 16) {
#pragma unroll
        for (int c = 0; c < HD / 16; ++c)
          *reinterpret_cast<u32x4*>(ctx_row + lhi * (HD / 2) + c * 8) = u32x4{0, 0, 0, 0};
      } else {
        *reinterpret_cast<u32x2*>(ctx_row + lhi * 4) = u32x2{0u, 0u};
      }
    }
    return;
  }

  int kv_end = kv_limit;
  if constexpr (CAUSAL) kv_end = min(kv_end, q0 + kBQ);
  const int nkb = (kv_end + kBKV - 1) / kBKV;

  const int64_t head_off = static_cast<int64_t>(bh) * S * HD;
  const bf16_t* Qh = Q + head_off;
  const bf16_t* Kh = Kg + head_off;
  const bf16_t* Vh = Vt + static_cast<int64_t>(bh) * HD * ld_vt;
  const uint8_t* Mh = (MASK == kMaskBytes) ? key_mask + static_cast<int64_t>(b) * S : nullptr;

  // Q fragments (B operand of S^T): lane (q = l32, k-group lhi) holds
  // d = 16*ks + 8*lhi .. +8.
  bf16x8 qf[kKSteps];
#pragma unroll
  for (int ks = 0; ks < kKSteps; ++ks) {
    if (qrow < S && (HD >= 16 || lhi == 0)) {
      qf[ks] = *reinterpret_cast<const bf16x8*>(Qh + static_cast<int64_t>(qrow) * HD + ks * 16 + lhi * 8);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) qf[ks][e] = static_cast<__bf16>(0.f);
    }
  }
  // MFMA row l32 of a 32-key block reads K row perm(l32)
  const int krow = 16 * ((l32 >> 3) >> 1) + 8 * ((l32 >> 2) & 1) + 4 * ((l32 >> 3) & 1) + (l32 & 3);

  // ---- tile loads ----
  // Full tiles: a load instruction fills 1 KiB of LDS, 64 lanes x 16 bytes in
  // lane order.  Load j of wavefront w covers slab NW j + w: K rows
  // (64 / (HD / 8)) slab .. +, lane L writing row first + L / (HD / 8), slot
  // L % (HD / 8); V^T rows 8 slab .. +7, lane L writing row 8 slab + L / 8,
  // slot L % 8.  Each lane fetches the chunk that its slot holds.
  // The loads are buffer loads on one resource per head for K and one for
  // V^T: a lane's byte offset inside its slab is fixed for the whole kernel
  // (computed here once), and the tile's position is a uniform soffset, so a
  // load costs no per-tile address arithmetic.  The host keeps one head's K
  // and V^T under 4 GiB (attention_seq_supported).
  constexpr int kLoadsPerWave = (kSlabs + NW - 1) / NW;
  const i32x4 k_rsrc = buffer_rsrc(Kh);
  const i32x4 v_rsrc = buffer_rsrc(Vh);
  int k_voff[kLoadsPerWave], v_voff[kLoadsPerWave];
#pragma unroll
  for (int j = 0; j < kLoadsPerWave; ++j) {
    const int slab = NW * j + wave;  // past kSlabs only when unused below
    const int rk = (kWave / kChunksK) * slab + lane / kChunksK;
    k_voff[j] = (rk * HD + ((lane % kChunksK) ^ k_swz<HD>(rk)) * 8) * 2;
    const int rv = 8 * slab + (lane >> 3);
    // (unsigned: a head's V^T may exceed 2 GiB)
    v_voff[j] = static_cast<int>((static_cast<uint32_t>(rv) * static_cast<uint32_t>(ld_vt) +
                                  static_cast<uint32_t>(((lane & 7) ^ v_swz(rv)) * 8)) * 2u);
  }
  auto issue_full = [&](int buf, int k0, bool with_v) {
#pragma unroll
    for (int j = 0; j < kLoadsPerWave; ++j) {
      const int slab = NW * j + wave;
      if (kSlabs % NW != 0 && slab >= kSlabs) break;  // uniform per wavefront
      const int rk0 = (kWave / kChunksK) * slab;
      enc_buffer_load_lds(k_rsrc, lds_ptr(&sK[buf * kTileElems + rk0 * HD]), 16, k_voff[j],
                          static_cast<int>(static_cast<uint32_t>(k0) * (HD * 2u)), 0, 0);
      if (with_v) {
        const int rv0 = 8 * slab;
        enc_buffer_load_lds(v_rsrc, lds_ptr(&sV[buf * kTileElems + rv0 * kBKV]), 16, v_voff[j], k0 * 2, 0, 0);
      }
    }
  };
  // The tile that crosses seq_len goes through registers: keys >= S read as
  // zeros (V^T's padding columns are never read, so they may hold anything).
  auto load_edge = [&](int buf, int k0, bool with_v) {
    for (int c = tid; c < kBKV * kChunksK; c += kThreads) {
      const int row = c / kChunksK, chunk = c % kChunksK;
      u32x4 kv = u32x4{0, 0, 0, 0};
      if (k0 + row < S) kv = *reinterpret_cast<const u32x4*>(Kh + static_cast<int64_t>(k0 + row) * HD + chunk * 8);
      *reinterpret_cast<u32x4*>(&sK[buf * kTileElems + k_off<HD>(row, chunk)]) = kv;
    }
    if (!with_v) return;
    for (int c = tid; c < HD * 8; c += kThreads) {
      const int row = c >> 3, chunk = c & 7;
      const int key = k0 + chunk * 8;
      const bf16_t* vp = Vh + static_cast<int64_t>(row) * ld_vt + key;
      uint16_t t[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) t[e] = (key + e < S) ? vp[e] : uint16_t(0);
      *reinterpret_cast<u32x4*>(&sV[buf * kTileElems + v_off(row, chunk)]) =
          u32x4{t[0] | (uint32_t(t[1]) << 16), t[2] | (uint32_t(t[3]) << 16),
                t[4] | (uint32_t(t[5]) << 16), t[6] | (uint32_t(t[7]) << 16)};
    }
  };
  auto issue_tile = [&](int buf, int kb, bool with_v) {
    const int k0 = kb * kBKV;
    if (k0 + kBKV <= S) {
      issue_full(buf, k0, with_v);
    } else {
      load_edge(buf, k0, with_v);
    }
    if constexpr (MASK == kMaskBytes) {
      if (tid < kBKV) sM[buf][tid] = (k0 + tid < S) ? Mh[k0 + tid] : uint8_t(0);
    }
  };

  // Runs body(buf, tile) over the first `active` of the nkb tiles in the
  // order 0, next(0), next(next(0)), ..., double-buffered: the loads of the
  // next tile overlap the current body.  The remaining tiles (a causal
  // wavefront's future) only take part in the loads and barriers the other
  // wavefronts need; keeping them out of the body's loop (rather than skipping
  // the body per tile) keeps the accumulators free of per-tile register
  // copies.  With resident tiles the body reads tile t from buffer t.
  bool resident = false;
  auto sweep = [&](auto next, bool with_v, int active, auto body) {
    if (RES > 0) {
      if (!resident) {
        for (int t = 0; t < nkb; ++t) issue_tile(t, t, true);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
        resident = true;
      }
      int tile = 0;
      for (int it = 0; it < active; ++it, tile = next(tile)) body(tile, tile);
    } else {
      int tile = 0;
      if (nkb > 0) issue_tile(0, tile, with_v);
      __builtin_amdgcn_s_waitcnt(kWaitVm0);
      __syncthreads();
      int it = 0;
      // Iteration `it` reads buffer it & 1.  For long rows the loop runs two
      // iterations per trip with the buffer index a constant in each, so the
      // bodies' LDS addresses fold into instruction offsets instead of being
      // recomputed per tile (c5 4%, c4 6% faster).  The warp-order bodies
      // (device expf) are twice as long: unrolled, the c3 kernel grew to
      // 64 KiB of code and ran 34% slower, so they keep one tile per trip.
      auto step = [&](auto cur_c) {
        constexpr int kCur = decltype(cur_c)::value;
        const int cur = kCur >= 0 ? kCur : (it & 1);
        const int nt = next(tile);
        if (it + 1 < nkb) issue_tile(cur ^ 1, nt, with_v);
        body(cur, tile);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
        tile = nt;
        ++it;
      };
      if constexpr (BLOCK_ORDER) {
        while (it + 1 < active) {
          step(std::integral_constant<int, 0>{});
          step(std::integral_constant<int, 1>{});
        }
        if (it < active) step(std::integral_constant<int, 0>{});  // it is even here
      } else {
        while (it < active) step(std::integral_constant<int, -1>{});
      }
      for (; it < nkb; ++it) {
        const int nt = next(tile);
        if (it + 1 < nkb) issue_tile((it & 1) ^ 1, nt, with_v);
        __builtin_amdgcn_s_waitcnt(kWaitVm0);
        __syncthreads();
        tile = nt;
      }
    }
  };

  const int wq_first = q0 + (kSplit ? 0 : wave * 32);
  const int wq_last = wq_first + 31;
  // tiles of the natural order this wavefront multiplies (causal: those with
  // a key <= its last query)
  const int active = CAUSAL ? min(nkb, wq_last / kBKV + 1) : nkb;

  // Raw fp32 dot products of the 64-key tile in LDS buffer `buf`.
  auto tile_dots = [&](int buf, f32x16 (&s)[2]) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      s[0][r] = 0.f;
      s[1][r] = 0.f;
    }
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
        const int chunk = HD >= 16 ? 2 * ks + lhi : 0;
        bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[buf * kTileElems + k_off<HD>(kb32 * 32 + krow, chunk)]);
        if (HD < 16 && lhi != 0) kf = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
        s[kb32] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], s[kb32], 0, 0, 0);
      }
    }
  };
  // Whether key (tile offset kl) is allowed for this lane's query.
  auto key_ok = [&](int buf, int k0, int kl) {
    const int key = k0 + kl;
    bool ok = key < kv_limit;
    if constexpr (CAUSAL) ok = ok && key <= qrow;
    if constexpr (MASK == kMaskBytes) ok = ok && sM[buf][kl] != 0;
    return ok;
  };
  auto tile_needs_mask = [&](int k0) {
    return (CAUSAL && k0 + kBKV - 1 > wq_first) || (k0 + kBKV > kv_limit) || (MASK == kMaskBytes);
  };
  // Score tile into s[2] as the softmax's first operation sees it:
  //   g = rn(s - max), s = bf16(bf16(q.k) * scale), excluded keys -inf.
  // With a power-of-two scale, s = bf16(q.k) * scale exactly and
  // rn(s - max) = scale * rn(bf16(q.k) - bf16(max raw dot)), so the scale
  // multiplies the difference (or folds into the exp2 multiplier below).
  // gap_scaled selects whether the returned g carries the scale.
  auto dots_to_gaps = [&](int buf, int k0, float row_max, float raw_max_bf, bool gap_scaled,
                          f32x16 (&s)[2]) {
#pragma unroll
    for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float v0 = round_bf16(s[kb32][r]), v1 = round_bf16(s[kb32][r + 1]);
        if constexpr (POW2_SCALE) {
          v0 = v0 - raw_max_bf;
          v1 = v1 - raw_max_bf;
          if (gap_scaled) {
            v0 *= scale;
            v1 *= scale;
          }
        } else {
          v0 = round_bf16(v0 * scale) - row_max;
          v1 = round_bf16(v1 * scale) - row_max;
        }
        s[kb32][r] = v0;
        s[kb32][r + 1] = v1;
      }
    }
    if (tile_needs_mask(k0)) {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          s[kb32][r] = key_ok(buf, k0, tile_key(kb32, r, lhi)) ? s[kb32][r] : -INFINITY;
    }
  };
  auto tile_gaps = [&](int buf, int k0, float row_max, float raw_max_bf, bool gap_scaled,
                       f32x16 (&s)[2]) {
    tile_dots(buf, s);
    dots_to_gaps(buf, k0, row_max, raw_max_bf, gap_scaled, s);
  };
  auto natural = [](int t) { return t + 1; };  // successor in key order
  // Rows of at most two tiles (RES == 2) keep each tile's values in registers
  // across the sweeps: the dot products of sweep A become the gaps and then
  // the weights e of sweep B, and sweep C reuses those e (the same values it
  // would recompute), so every score's exponential is evaluated once.
  constexpr bool kCache = RES == 2;
  f32x16 cache[kCache && !kSplit ? 2 : 1][2];
  auto load_resident = [&]() {
    for (int t = 0; t < nkb; ++t) issue_tile(t, t, true);
    __builtin_amdgcn_s_waitcnt(kWaitVm0);
    __syncthreads();
  };

  // ============================ sweep A: row max ============================
  // max (and, for the short-row regime, min) of the raw dot products of the
  // allowed keys; the bf16 score of the max is formed once afterwards.
  // Long rows use the NaN-propagating maximum (v_maximum3_f32), which needs
  // no NaN-quieting copy of each MFMA result as fmaxf does; for numbers the
  // two agree except in the sign of a zero max, which changes no gap's value
  // (s - (+0) = s - (-0), and exp(-0) = exp(+0) = 1).  (Short rows keep
  // fmaxf / fminf: no gain was measured there.)
  float mx = -INFINITY, mn = INFINITY;
  auto vmax = [](float a, float b) {
    if constexpr (BLOCK_ORDER) {
      return __builtin_elementwise_maximum(a, b);
    } else {
      return fmaxf(a, b);
    }
  };
  auto vmin = [](float a, float b) { return fminf(a, b); };
  auto max_body = [&](int buf, int kb, f32x16 (&s)[2]) {
    const int k0 = kb * kBKV;
    tile_dots(buf, s);
    if (tile_needs_mask(k0)) {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const bool ok = key_ok(buf, k0, tile_key(kb32, r, lhi));
          mx = vmax(mx, ok ? s[kb32][r] : -INFINITY);
          if constexpr (!BLOCK_ORDER) mn = vmin(mn, ok ? s[kb32][r] : INFINITY);
        }
      }
    } else {
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        mx = vmax(mx, vmax(vmax(s[0][r], s[0][r + 1]), vmax(s[1][r], s[1][r + 1])));
        if constexpr (!BLOCK_ORDER) mn = vmin(mn, vmin(vmin(s[0][r], s[0][r + 1]), vmin(s[1][r], s[1][r + 1])));
      }
    }
  };
  if constexpr (kSplit) {
    load_resident();
    if (wave < active) max_body(wave, wave, cache[0]);
  } else if constexpr (kCache) {
    load_resident();
#pragma unroll
    for (int t = 0; t < 2; ++t)
      if (t < active) max_body(t, t, cache[t]);
  } else {
    sweep(natural, false, active, [&](int buf, int kb) {
      f32x16 s[2];
      max_body(buf, kb, s);
    });
  }
  mx = fmaxf(mx, __shfl_xor(mx, 32, kWave));
  if constexpr (kSplit) {
    mn = fminf(mn, __shfl_xor(mn, 32, kWave));
    x_mm[wave * kWave + lane] = mx;
    x_mm[(2 + wave) * kWave + lane] = mn;
    __syncthreads();
    mx = fmaxf(x_mm[lane], x_mm[kWave + lane]);
    mn = fminf(x_mm[2 * kWave + lane], x_mm[3 * kWave + lane]);
  }
  auto to_score = [&](float raw) {
    const float rq = round_bf16(raw);
    return POW2_SCALE ? rq * scale : round_bf16(rq * scale);
  };
  const float row_max = (mx == -INFINITY) ? -INFINITY : to_score(mx);
  const float raw_max_bf = (mx == -INFINITY) ? -INFINITY : round_bf16(mx);
  // exp2 multiplier of the long-row regime: log2(e), times the scale when the
  // gap is kept unscaled (exact: the scale is a power of two)
  const float c_exp = POW2_SCALE ? scale * kLog2e : kLog2e;
  bool slow_div = false;
  if constexpr (!BLOCK_ORDER) {
    mn = fminf(mn, __shfl_xor(mn, 32, kWave));
    // weights below 2^-100 could underflow inside the Markstein quotient
    const bool tiny = (mn != INFINITY) && (to_score(mn) - row_max < kMinFastGap);
    slow_div = __builtin_amdgcn_ballot_w64(tiny) != 0;
  }
  // Gaps -> weights exp(gap) in place (short-row regime).  Without the fast
  // division verdict's exception (slow_div) every allowed key's gap is at
  // least kMinFastGap, and a tile with no excluded key holds no -inf, so the
  // underflow clamp (below -103.28) cannot fire there and is left out.
  // exp(s - max) of a gap in the short-row regime.  With a power-of-two
  // scale the gaps stay unscaled (g = bf16(q.k) - bf16(max raw dot)) and the
  // scale is folded into expf's constants: the same bits as expf(g * scale),
  // one multiply fewer per score.
  const ExpfScaled ec = expf_scaled_consts(scale);
  auto exp_gap = [&](float g) { return kFoldScale ? expf_nonpos_scaled(g, ec) : expf_nonpos(g); };
  auto exp_gap_unclamped = [&](float g) {
    return kFoldScale ? expf_nonpos_scaled_unclamped(g, ec) : expf_nonpos_unclamped(g);
  };
  auto tile_exp = [&](f32x16 (&s)[2], bool clamp) {
    if (clamp) {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb32][r] = exp_gap(s[kb32][r]);
    } else {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int r = 0; r < 16; ++r) s[kb32][r] = exp_gap_unclamped(s[kb32][r]);
    }
  };

  // One 32-key half (kb32) of a tile: the half's q.k chain over the head dim
  // and its scores as the softmax's first operation sees them (gaps, excluded
  // keys -inf): tile_dots and dots_to_gaps for half of the scores.
  auto gaps_half = [&](int buf, int k0, int kb32, bool masked, f32x16& sh) __attribute__((always_inline)) {
#pragma unroll
    for (int r = 0; r < 16; ++r) sh[r] = 0.f;
#pragma unroll
    for (int ks = 0; ks < kKSteps; ++ks) {
      const int chunk = HD >= 16 ? 2 * ks + lhi : 0;
      bf16x8 kf = *reinterpret_cast<const bf16x8*>(&sK[buf * kTileElems + k_off<HD>(kb32 * 32 + krow, chunk)]);
      if (HD < 16 && lhi != 0) kf = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
      sh = __builtin_amdgcn_mfma_f32_32x32x16_bf16(kf, qf[ks], sh, 0, 0, 0);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      float v = round_bf16(sh[r]);
      if constexpr (POW2_SCALE) {
        v = v - raw_max_bf;
        if (!kFoldScale) v *= scale;
      } else {
        v = round_bf16(v * scale) - row_max;
      }
      sh[r] = v;
    }
    if (masked) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sh[r] = key_ok(buf, k0, tile_key(kb32, r, lhi)) ? sh[r] : -INFINITY;
    }
  };
  // sweep B on one half: its 16 weights added to their partials
  // (The weights replace the gaps in place under the branch and are added
  // after it: with the adds inside the two paths, both halves' partials were
  // copied between registers at the join, 32 moves per half.)
  auto sum_half = [&](int buf, int k0, int kb32, bool masked, bool clamp, float (&p)[16]) __attribute__((always_inline)) {
    f32x16 sh;
    gaps_half(buf, k0, kb32, masked, sh);
    if (clamp) {
#pragma unroll
      for (int r = 0; r < 16; ++r) sh[r] = exp_gap(sh[r]);
    } else {
#pragma unroll
      for (int r = 0; r < 16; ++r) sh[r] = exp_gap_unclamped(sh[r]);
    }
#pragma unroll
    for (int r = 0; r < 16; ++r) p[r] += sh[r];
  };

  // ======================= sweep B: row sum of exp(s - max) =======================
  float row_sum;
  if constexpr (!BLOCK_ORDER) {
    // warp order: partial[lam] over keys lam, lam+64, ... (lam = key % 64)
    float part[2][16];
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      part[0][r] = 0.f;
      part[1][r] = 0.f;
    }
    if constexpr (kSplit) {
      // this wavefront's weights, zeros for a tile no query of the block sees
      if (wave < active) {
        dots_to_gaps(wave, wave * kBKV, row_max, raw_max_bf, !kFoldScale, cache[0]);
        tile_exp(cache[0], slow_div || tile_needs_mask(wave * kBKV));
      } else {
#pragma unroll
        for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
          for (int r = 0; r < 16; ++r) cache[0][kb32][r] = 0.f;
      }
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int r = 0; r < 16; ++r) x_e[(wave * 32 + kb32 * 16 + r) * kWave + lane] = cache[0][kb32][r];
      __syncthreads();
      // partial = e(tile 0) + e(tile 1), the order of the one-wavefront loop
      // (0 + e0 = e0 exactly, and an unseen tile adds +0)
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
        for (int r = 0; r < 16; ++r)
          part[kb32][r] = x_e[(kb32 * 16 + r) * kWave + lane] + x_e[(32 + kb32 * 16 + r) * kWave + lane];
    } else if constexpr (kCache) {
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        if (t >= active) continue;
        dots_to_gaps(t, t * kBKV, row_max, raw_max_bf, !kFoldScale, cache[t]);
        tile_exp(cache[t], slow_div || tile_needs_mask(t * kBKV));
#pragma unroll
        for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
          for (int r = 0; r < 16; ++r) part[kb32][r] += cache[t][kb32][r];
      }
    } else if constexpr (kHalfTiles) {
      sweep(natural, false, active, [&](int buf, int kb) {
        const int k0 = kb * kBKV;
        const bool masked = tile_needs_mask(k0);
        sum_half(buf, k0, 0, masked, slow_div || masked, part[0]);
        sum_half(buf, k0, 1, masked, slow_div || masked, part[1]);
      });
    } else {
      sweep(natural, false, active, [&](int buf, int kb) {
        const int k0 = kb * kBKV;
        f32x16 s[2];
        tile_gaps(buf, k0, row_max, raw_max_bf, !kFoldScale, s);
        tile_exp(s, slow_div || tile_needs_mask(k0));
#pragma unroll
        for (int kb32 = 0; kb32 < 2; ++kb32)
#pragma unroll
          for (int r = 0; r < 16; ++r) part[kb32][r] += s[kb32][r];
      });
    }
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
    // visited residue-major; "warp" w covers residues 4w .. 4w+3.  All partial
    // arrays are indexed statically: the running residue's partials live in
    // acc[]; of a warp's finished residues r0..r3, r0 goes to h0 and r1 to h1,
    // r2 is added to h0 as it finishes (r0 + r2, the tree's first pair), and
    // r3 completes the warp: (r0 + r2) + (r1 + r3).  A finished warp's sum is
    // shifted into warp_sum[].
    // successor in residue-major order: tiles r, r + 32, r + 64, ..., then r + 1
    auto resmajor = [&](int t) { return t + 32 < nkb ? t + 32 : (t & 31) + 1; };
    float warp_sum[8];
    float h0[8], h1[8];  // the current warp's finished residues (see above)
    float acc[8];        // [vector slot 4*kb32 + i] of the running residue
#pragma unroll
    for (int w = 0; w < 8; ++w) warp_sum[w] = 0.f;
#pragma unroll
    for (int v = 0; v < 8; ++v) {
      acc[v] = 0.f;
      h0[v] = 0.f;
      h1[v] = 0.f;
    }
    int cur_res = 0;
    // residue cur_res is complete: file it (uniform branch on its position in
    // the warp); after a warp's fourth residue, reduce the warp with a
    // shuffle-down tree over lam = 16 rr + u, u = 8 kb32 + 4 (i>>1) + 2 h + (i&1):
    // offsets 32, 16 (rr), 8 (kb32), 4 (i>>1), 2 (lane half), 1 (i&1)
    auto finish_residue = [&]() {
      const int q = cur_res & 3;
      ++cur_res;
      if (q == 0) {
#pragma unroll
        for (int v = 0; v < 8; ++v) h0[v] = acc[v];
      } else if (q == 1) {
#pragma unroll
        for (int v = 0; v < 8; ++v) h1[v] = acc[v];
      } else if (q == 2) {
#pragma unroll
        for (int v = 0; v < 8; ++v) h0[v] = h0[v] + acc[v];
      } else {
        float t8[8];
#pragma unroll
        for (int v = 0; v < 8; ++v) t8[v] = h0[v] + (h1[v] + acc[v]);
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
        for (int w = 0; w < 7; ++w) warp_sum[w] = warp_sum[w + 1];
        warp_sum[7] = ws;
      }
#pragma unroll
      for (int v = 0; v < 8; ++v) acc[v] = 0.f;
    };
    sweep(resmajor, false, nkb, [&](int buf, int kb) {
      const int k0 = kb * kBKV;
      const int r = kb & 31;
      // Every residue below min(32, nkb) owns a tile, so in residue-major
      // order the next tile is either the current residue's or the next
      // one's: at most one residue finishes here (an `if`, not a loop, which
      // spares the register copies a loop-carried accumulator costs); the
      // residues with no tile finish after the sweep.
      if (cur_res < r) finish_residue();  // uniform
      if (CAUSAL && k0 > wq_last) return;
      f32x16 s[2];
      tile_gaps(buf, k0, row_max, raw_max_bf, false, s);
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          float a = acc[4 * kb32 + i];
#pragma unroll
          for (int j = 0; j < 4; ++j) a += __builtin_amdgcn_exp2f(s[kb32][4 * i + j] * c_exp);
          acc[4 * kb32 + i] = a;
        }
      }
    });
    while (cur_res < 32) finish_residue();
    // tree over the 8 warp sums (offsets 4, 2, 1)
    const float a0 = warp_sum[0] + warp_sum[4], a1 = warp_sum[1] + warp_sum[5];
    const float a2 = warp_sum[2] + warp_sum[6], a3 = warp_sum[3] + warp_sum[7];
    row_sum = (a0 + a2) + (a1 + a3);
  }

  // ================== sweep C: p = bf16(softmax), context += P V ==================
  // Correctly rounded 1 / sum: the block-order epilogue multiplies by it; the
  // short-row regime uses it as the Markstein reciprocal.
  const float inv_sum = 1.0f / row_sum;
  f32x16 o[kDBlocks];
#pragma unroll
  for (int db = 0; db < kDBlocks; ++db)
#pragma unroll
    for (int r = 0; r < 16; ++r) o[db][r] = 0.f;
  // s holds the gaps, or (have_e) the weights e themselves
  auto make_pf = [&](f32x16 (&s)[2], bool have_e, bf16x8 (&pf)[4]) {
    if (BLOCK_ORDER || !slow_div) {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = have_e ? s[kb32][r]
                          : BLOCK_ORDER ? __builtin_amdgcn_exp2f(s[kb32][r] * c_exp) : exp_gap(s[kb32][r]);
          float p;
          if constexpr (BLOCK_ORDER) {
            p = e * inv_sum;
          } else {
            const float q = e * inv_sum;
            p = fmaf(fmaf(-q, row_sum, e), inv_sum, q);
          }
          pf[kb32 * 2 + (r >> 3)][r & 7] = static_cast<__bf16>(p);
        }
      }
    } else {
#pragma unroll
      for (int kb32 = 0; kb32 < 2; ++kb32) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const float e = have_e ? s[kb32][r] : exp_gap(s[kb32][r]);
          pf[kb32 * 2 + (r >> 3)][r & 7] = static_cast<__bf16>(e / row_sum);
        }
      }
    }
  };
  auto pv_mfma = [&](int buf, const bf16x8 (&pf)[4]) {
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
        const int vrow = HD >= 32 ? db * 32 + l32 : (l32 & (HD - 1));
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&sV[buf * kTileElems + v_off(vrow, 2 * kk + lhi)]);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf[kk], o[db], 0, 0, 0);
      }
    }
  };
  auto pv_body = [&](int buf, f32x16 (&s)[2], bool have_e) {
    bf16x8 pf[4];
    make_pf(s, have_e, pf);
    pv_mfma(buf, pf);
  };
  // Sweep C on one half (kHalfTiles): its weights, its two P fragments and
  // their P.V MFMAs (kk = 2 kb32, 2 kb32 + 1), the whole tile's chain order.
  auto pv_half = [&](int buf, int k0, int kb32, bool masked, bool slow) __attribute__((always_inline)) {
    f32x16 sh;
    gaps_half(buf, k0, kb32, masked, sh);
    bf16x8 pf2[2];
    if (slow) {
#pragma unroll
      for (int r = 0; r < 16; ++r) pf2[r >> 3][r & 7] = static_cast<__bf16>(exp_gap(sh[r]) / row_sum);
    } else {
      if (masked) {
#pragma unroll
        for (int r = 0; r < 16; ++r) sh[r] = exp_gap(sh[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 16; ++r) sh[r] = exp_gap_unclamped(sh[r]);
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const float e = sh[r];
        const float q = e * inv_sum;
        const float p = fmaf(fmaf(-q, row_sum, e), inv_sum, q);
        pf2[r >> 3][r & 7] = static_cast<__bf16>(p);
      }
    }
#pragma unroll
    for (int h2 = 0; h2 < 2; ++h2) {
      const int kk = 2 * kb32 + h2;
#pragma unroll
      for (int db = 0; db < kDBlocks; ++db) {
        const int vrow = HD >= 32 ? db * 32 + l32 : (l32 & (HD - 1));
        const bf16x8 vf = *reinterpret_cast<const bf16x8*>(&sV[buf * kTileElems + v_off(vrow, 2 * kk + lhi)]);
        o[db] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(vf, pf2[h2], o[db], 0, 0, 0);
      }
    }
  };
  if constexpr (kSplit) {
    bf16x8 pf[4];
    if (wave < active) make_pf(cache[0], true, pf);
    if (wave == 1 && active > 1) {
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) x_p[lane * 4 + kk] = pf[kk];
    }
    __syncthreads();
    if (wave == 1) return;
    if (active > 0) pv_mfma(0, pf);
    if (active > 1) {
      bf16x8 pf1[4];
#pragma unroll
      for (int kk = 0; kk < 4; ++kk) pf1[kk] = x_p[lane * 4 + kk];
      pv_mfma(1, pf1);
    }
  } else if constexpr (kCache) {
#pragma unroll
    for (int t = 0; t < 2; ++t)
      if (t < active) pv_body(t, cache[t], true);
  } else if constexpr (kHalfTiles) {
    if (!slow_div) {
      sweep(natural, true, active, [&](int buf, int kb) {
        const int k0 = kb * kBKV;
        const bool masked = tile_needs_mask(k0);
        pv_half(buf, k0, 0, masked, false);
        pv_half(buf, k0, 1, masked, false);
      });
    } else {
      sweep(natural, true, active, [&](int buf, int kb) {
        const int k0 = kb * kBKV;
        const bool masked = tile_needs_mask(k0);
        pv_half(buf, k0, 0, masked, true);
        pv_half(buf, k0, 1, masked, true);
      });
    }
  } else if constexpr (!BLOCK_ORDER) {
    // One loop per division form (fixed for the row): with the choice inside
    // the loop the two paths' P.V chains left the accumulators in different
    // registers, copied back every tile.
    if (!slow_div) {
      sweep(natural, true, active, [&](int buf, int kb) {
        f32x16 s[2];
        tile_gaps(buf, kb * kBKV, row_max, raw_max_bf, !kFoldScale, s);
        tile_exp(s, tile_needs_mask(kb * kBKV));
        pv_body(buf, s, true);
      });
    } else {
      sweep(natural, true, active, [&](int buf, int kb) {
        f32x16 s[2];
        tile_gaps(buf, kb * kBKV, row_max, raw_max_bf, !kFoldScale, s);
        pv_body(buf, s, false);
      });
    }
  } else {
    sweep(natural, true, active, [&](int buf, int kb) {
      f32x16 s[2];
      tile_gaps(buf, kb * kBKV, row_max, raw_max_bf, false, s);
      pv_body(buf, s, false);
    });
  }

  // ---- write context[b, qrow, h*HD + d] = bf16(O) ----
  if (qrow < S) {
    bool zero = !(row_sum > 0.f);
    if constexpr (MASK == kMaskPrefix) zero = zero || qrow >= kv_limit;
#pragma unroll
    for (int db = 0; db < kDBlocks; ++db) {
#pragma unroll
      for (int i = 0; i < (HD < 32 ? HD / 8 : 4); ++i) {
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

// LDS bytes of one attention workgroup: K and V^T tiles plus key-mask bytes,
// and with the key split (two wavefronts) the exchange areas
constexpr size_t attn_lds_bytes(int hd, int res, bool split = false) {
  const size_t tiles = static_cast<size_t>(res > 0 ? res : 2) * (2 * kBKV * hd * sizeof(bf16_t) + kBKV);
  if (!split) return tiles;
  return (tiles + 15) / 16 * 16 + (2 * 2 * kWave + 2 * 32 * kWave) * sizeof(float) + kWave * 4 * 16;
}

template <int HD, int NW, bool CAUSAL, int MASK, bool POW2, bool BLOCK_ORDER, int RES = 0, int OCC = 1>
hipError_t launch_attn(const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B,
                       int H, int S, float scale, const int32_t* kv_len, const uint8_t* key_mask,
                       hipStream_t st) {
  constexpr bool kSplit = NW == 2 && RES == 2;
  constexpr int kBQ = kSplit ? 32 : NW * 32;
  constexpr size_t kLds = attn_lds_bytes(HD, RES, kSplit);
  const int nqb = (S + kBQ - 1) / kBQ;
  const dim3 grid(static_cast<uint32_t>(B) * H * nqb);
  const int ld_vt = static_cast<int>(vt_stride(S));
  auto kernel = attn_fwd_kernel<HD, NW, CAUSAL, MASK, POW2, BLOCK_ORDER, RES, OCC>;
  if constexpr (kLds > 64 * 1024) {
    // above 64 KiB of dynamic LDS the kernel has to opt in (once per process)
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       static_cast<int>(kLds));
    if (attr != hipSuccess) return attr;
  }
  hipLaunchKernelGGL(kernel, grid, dim3(NW * kWave), kLds, st, q, k, vt, ctx, H, S, ld_vt, nqb, scale, kv_len,
                     key_mask);
  return hipGetLastError();
}

template <int HD, bool CAUSAL, int MASK, bool POW2>
hipError_t dispatch_order(const bf16_t* q, const bf16_t* k, const bf16_t* vt, bf16_t* ctx, int B,
                          int H, int S, float scale, const int32_t* kv_len,
                          const uint8_t* key_mask, hipStream_t st) {
  if (S > kWarpSoftmaxMaxKeys) {
    // Long rows: with at least four workgroups per CU to run, head dim 64
    // without a byte mask asks for four wavefronts per SIMD instead of the
    // three its unconstrained allocation allows (measured 4% faster on 8192
    // causal keys, 2% on 100000 keys).  Smaller grids cannot use the extra
    // residency and would only pay for the spills (12% slower at 198
    // workgroups); the byte-mask form would spill 18 registers at that bound.
    if constexpr (HD == 64 && MASK != kMaskBytes) {
      const int64_t groups = static_cast<int64_t>(B) * H * ((S + 127) / 128);
      if (groups >= 4 * 256)
        return launch_attn<HD, 4, CAUSAL, MASK, POW2, true, 0, 4>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
    }
    return launch_attn<HD, 4, CAUSAL, MASK, POW2, true>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  }
  // Small problems use workgroups of 32 queries (one wavefront, or two that
  // split the keys) so more of the 256 CUs get work; larger ones share each
  // K/V tile among 4 wavefronts.
  // Rows of at most 256 keys keep every tile resident in LDS (at most 128 keys
  // for head dim 256, whose four resident tiles would exceed the 160 KiB of
  // LDS of a CU).
  constexpr bool kRes4 = attn_lds_bytes(HD, 4) <= 160 * 1024;
  const int64_t groups128 = static_cast<int64_t>(B) * H * ((S + 127) / 128);
  if (groups128 < 512) {
    // rows of at most 128 keys: two wavefronts per 32 queries (key split)
    if (S <= 2 * kBKV)
      return launch_attn<HD, 2, CAUSAL, MASK, POW2, false, 2>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
    if constexpr (kRes4) {
      if (S <= 4 * kBKV)
        return launch_attn<HD, 1, CAUSAL, MASK, POW2, false, 4>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
    }
    return launch_attn<HD, 1, CAUSAL, MASK, POW2, false>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  }
  if (S <= 2 * kBKV)
    return launch_attn<HD, 4, CAUSAL, MASK, POW2, false, 2>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  if constexpr (kRes4) {
    if (S <= 4 * kBKV)
      return launch_attn<HD, 4, CAUSAL, MASK, POW2, false, 4>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  }
  // Head dim 64: three wavefronts per SIMD with the half-tile sweeps where
  // they measured faster (H = 16, one process, bitwise the same): causal
  // without key masks (B = 8: S = 1024 103.9 -> 93.2 us, S = 777 72.6 ->
  // 63.6; B = 16, S = 300 38.7 -> 30.3; B = 4, S = 2048 153.8 -> 148.1) and
  // non-causal rows of more than 512 keys with or without a prefix mask
  // (B = 8, S = 1024: 144.1 -> 137.9, prefix 134.5 -> 128.5).  The
  // two-wavefront kernel stays for causal prefix masks (S = 1000: 68.6 vs
  // 77.3), byte masks (S = 900: 138.9 vs 144.6) and non-causal rows of up to
  // 512 keys (40.9 vs 42.0).
  if constexpr (HD == 64 && MASK != kMaskBytes && !(CAUSAL && MASK == kMaskPrefix)) {
    if (CAUSAL || S > 512)
      return launch_attn<HD, 4, CAUSAL, MASK, POW2, false, 0, 3>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  }
  return launch_attn<HD, 4, CAUSAL, MASK, POW2, false>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

template <int HD, bool CAUSAL, int MASK>
hipError_t dispatch_pow2(bool pow2, const bf16_t* q, const bf16_t* k, const bf16_t* vt,
                         bf16_t* ctx, int B, int H, int S, float scale, const int32_t* kv_len,
                         const uint8_t* key_mask, hipStream_t st) {
  // The general path evaluates bf16(bf16(q.k) * scale) literally, which is
  // exact for every scale; the power-of-two variant only saves work.  Head
  // dims other than 64 instantiate the general one only.
  if constexpr (HD == 64) {
    if (pow2) return dispatch_order<HD, CAUSAL, MASK, true>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  }
  (void)pow2;
  return dispatch_order<HD, CAUSAL, MASK, false>(q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

template <int HD, bool CAUSAL>
hipError_t dispatch_mask(int mask, bool pow2, const bf16_t* q, const bf16_t* k, const bf16_t* vt,
                         bf16_t* ctx, int B, int H, int S, float scale, const int32_t* kv_len,
                         const uint8_t* key_mask, hipStream_t st) {
  if (mask == kMaskPrefix) return dispatch_pow2<HD, CAUSAL, kMaskPrefix>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  if (mask == kMaskBytes) return dispatch_pow2<HD, CAUSAL, kMaskBytes>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
  return dispatch_pow2<HD, CAUSAL, kMaskNone>(pow2, q, k, vt, ctx, B, H, S, scale, kv_len, key_mask, st);
}

// Exact attention at head_dim HD: argument checks are the caller's.
template <int HD>
hipError_t exact_attention(const bf16_t* q, const bf16_t* k, const bf16_t* v_t, bf16_t* ctx, int batch,
                           int heads, int seq_len, float scale, const int32_t* kv_len,
                           const uint8_t* key_mask, bool causal, hipStream_t stream) {
  int mant_exp = 0;
  const float mant = frexpf(scale, &mant_exp);
  const bool pow2 = (mant == 0.5f);
  const int mask = key_mask != nullptr ? kMaskBytes : (kv_len != nullptr ? kMaskPrefix : kMaskNone);
  if (causal)
    return dispatch_mask<HD, true>(mask, pow2, q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask,
                                   stream);
  return dispatch_mask<HD, false>(mask, pow2, q, k, v_t, ctx, batch, heads, seq_len, scale, kv_len, key_mask,
                                  stream);
}

}  // namespace

}  // namespace enc
