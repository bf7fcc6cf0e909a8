// bf16 MFMA GEMM with fused nn.Linear epilogues for gfx950.
//
//   C[M, N] = epilogue(A[M, K] . W[N, K]^T + bias)
//
// A (activations) and W (nn.Linear weight, [out, in]) are both K-contiguous,
// so both tiles are staged in LDS the same way: [rows][BK + 8] bf16, the 8-element
// pad (16 bytes) spreading the 16-byte MFMA operand reads of 32 consecutive rows
// across all LDS banks.
//
// Work decomposition: 256 threads = 4 wavefronts in a 2 x 2 grid; each
// wavefront owns a (BM/2) x (BN/2) sub-tile computed with
// v_mfma_f32_32x32x16_bf16 (fp32 accumulators).  The K loop double-buffers LDS:
// the global loads of tile k+1 are issued before the MFMAs of tile k and are
// written to the other LDS buffer afterwards, so one barrier per K step suffices.
//
// MFMA 32x32x16 operand/accumulator lane layout (lane l, 0..63):
//   A operand : row l%32, k = 8*(l/32) + e   (e = 0..7)
//   B operand : col l%32, k = 8*(l/32) + e
//   C/D       : col l%32, row = 8*(r/4) + 4*(l/32) + r%4   (r = 0..15)
//
// Workgroup -> tile mapping is XCD-aware: MI355X dispatches consecutive
// workgroups round-robin over its 8 XCDs, so the linear id is remapped so each
// XCD walks a contiguous range of tiles, which are ordered in groups of 8 tile
// rows so concurrently running tiles share A rows and W columns in that XCD's L2.
#include <algorithm>
#include <mutex>
#include <vector>

#include "common.h"
#include "kernels.h"
#include "streamk_tail.h"

namespace enc {

namespace {

constexpr int kBK = 64;
constexpr int kLdk = kBK + 8;  // padded LDS row, elements
constexpr int kThreads = 256;
constexpr int kNumXcd = 8;
constexpr int kGroupM = 8;

__device__ __forceinline__ void map_tile(int tiles_m, int tiles_n, int pid, int* tm, int* tn) {
  const int num = tiles_m * tiles_n;
  // XCD remap: workgroups pid = x + 8*slot run on XCD x.
  {
    const int xcd = pid % kNumXcd;
    const int slot = pid / kNumXcd;
    const int base = num / kNumXcd;
    const int rem = num % kNumXcd;
    pid = xcd * base + min(xcd, rem) + slot;
  }
  const int per_group = kGroupM * tiles_n;
  const int group = pid / per_group;
  const int first_m = group * kGroupM;
  const int group_m = min(tiles_m - first_m, kGroupM);
  const int in_group = pid % per_group;
  *tm = first_m + in_group % group_m;
  *tn = in_group / group_m;
}

// torch's exact GELU of every bf16 value, bf16(gelu_erf(x)) for all 65536 bit
// patterns x: the input of a GELU epilogue is the bf16 nn.Linear output, so
// one lookup gives the same bits as the erf evaluation.  Each device's table
// is filled by gelu_table_kernel, after which gelu_ready_kernel sets
// g_gelu_ready on the same stream; an epilogue that finds the flag clear
// (a product on another stream racing the first fill, or a cached copy of
// the flag from before it was set) evaluates the erf instead, which gives the
// same bits.
__device__ __attribute__((aligned(256))) uint16_t g_gelu_table[65536];
__device__ uint32_t g_gelu_ready;

__global__ void __launch_bounds__(256) gelu_table_kernel() {
  const uint32_t x = blockIdx.x * 256u + threadIdx.x;
  g_gelu_table[x] = f32_to_bf16(gelu_erf(__uint_as_float(x << 16)));
}

__global__ void gelu_ready_kernel() {
  __hip_atomic_store(&g_gelu_ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Test hooks: set the ready flag, and overwrite (value >= 0) or recompute
// (value < 0) one table entry.
__global__ void gelu_flag_set_kernel(uint32_t ready) {
  __hip_atomic_store(&g_gelu_ready, ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

__global__ void gelu_entry_set_kernel(uint32_t x, int32_t value) {
  g_gelu_table[x] = value < 0 ? f32_to_bf16(gelu_erf(__uint_as_float(x << 16))) : static_cast<uint16_t>(value);
}

// The wide kernel's GELU epilogue reads a compact copy of the table from LDS:
// for each sign, the bf16 magnitudes a = bits & 0x7fff in [kGeluLo, kGeluHi]
// (|x| from 2.4e-4 to 5.53; 7.2 KiB for both signs, which leaves two 256x128
// workgroups per CU room).  Outside that range the values follow from x
// itself, as torch's GELU of every bf16 pattern shows (checked exhaustively):
//   a < kGeluLo:  bf16(0.5 x)  (erf(x / sqrt 2) is below half an ulp of 1);
//   a > kGeluHi:  x for x > 0, -0 for x < 0, the canonical NaN 0x7fc0 for
//                 NaN inputs and for -inf (-inf * 0).
// The table region is filled from g_gelu_table's two slices (the entries for
// a positive x are x itself from 2.77 on).  A pass whose eight values all lie
// in the range (nearly every pass for activations of unit scale) does only the
// lookups; otherwise the pass evaluates the rules above per value.
constexpr uint32_t kGeluLo = 0x3980u;
constexpr uint32_t kGeluHi = 0x40b1u;
constexpr int kGeluSpan = static_cast<int>(kGeluHi - kGeluLo + 1);  // entries per sign
static_assert(kGeluSpan % 2 == 0 && kGeluLo % 2 == 0, "whole 4-byte words per slice");

// GELU of one bf16 pattern u through the compact table (any u)
__device__ __forceinline__ uint32_t gelu_compact(const bf16_t* tab, uint32_t u) {
  const uint32_t a = u & 0x7fffu, s = u >> 15;
  const uint32_t c = min(max(a, kGeluLo), kGeluHi);
  const uint32_t t = tab[s * kGeluSpan + (c - kGeluLo)];
  const uint32_t half = f32_to_bf16(__uint_as_float(u << 16) * 0.5f);
  const uint32_t big = (a + s > 0x7f80u) ? 0x7fc0u : (s != 0u ? 0x8000u : u);
  return a < kGeluLo ? half : (a > kGeluHi ? big : t);
}

// 8 GELU outputs of 8 bf16 values (two per word, low half first)
__device__ __forceinline__ u32x4 gelu8_lds(const bf16_t* tab, u32x4 v) {
  uint32_t u[8];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    u[2 * e] = v[e] & 0xffffu;
    u[2 * e + 1] = v[e] >> 16;
  }
  bool in_range = true;
#pragma unroll
  for (int e = 0; e < 8; ++e) in_range = in_range && (u[e] & 0x7fffu) - kGeluLo <= kGeluHi - kGeluLo;
  uint32_t g[8];
  if (__builtin_amdgcn_ballot_w64(!in_range) == 0) {
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = tab[(u[e] >> 15) * kGeluSpan + ((u[e] & 0x7fffu) - kGeluLo)];
  } else {
#pragma unroll
    for (int e = 0; e < 8; ++e) g[e] = gelu_compact(tab, u[e]);
  }
  return u32x4{g[0] | (g[1] << 16), g[2] | (g[3] << 16), g[4] | (g[5] << 16), g[6] | (g[7] << 16)};
}


template <int EPI>
__device__ __forceinline__ void store_row_major(const GemmEpilogueArgs& ep, int N, int row,
                                                int col, float acc, float bias) {
  const int64_t idx = static_cast<int64_t>(row) * N + col;
  const float y = round_bf16(acc + bias);  // nn.Linear output boundary
  if constexpr (EPI == kEpiBias) {
    ep.out[idx] = f32_to_bf16(y);
  } else if constexpr (EPI == kEpiBiasGelu) {
    ep.out[idx] = f32_to_bf16(gelu_erf(y));
  } else {
    const bf16_t r = ep.residual[idx];
    bool keep = true;
    if (ep.row_mask != nullptr) keep = ep.row_mask[row] != 0;
    if (keep) {
      ep.out[idx] = f32_to_bf16(bf16_to_f32(r) + y);
    } else {
      ep.out[idx] = (EPI == kEpiResidualKeep) ? r : bf16_t(0);
    }
  }
}

// Writes one 32x32 fp32 accumulator block (rows row0.., cols col0..) through
// the epilogue.  Lane l holds column col0 + l%32, rows 8*(r/4) + 4*(l/32) + r%4.
template <int EPI>
__device__ __forceinline__ void store_block(const GemmEpilogueArgs& ep, int M, int N, int row0,
                                            int col0, const f32x16& acc) {
  const int lane = threadIdx.x % kWave;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;
  const int col = col0 + l32;
  const float bias = bf16_to_f32(ep.bias[col]);
  if constexpr (EPI == kEpiQkvHeadMajor) {
    const int D = ep.d_model;
    const int hd = ep.head_dim;
    const int which = col / D;
    const int rem = col - which * D;
    const int h = rem / hd;
    const int d = rem - h * hd;
    const int S = ep.seq_len;
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int r0 = row0 + 8 * g + 4 * lhi;  // 4 consecutive rows
      float y[4];
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) y[jj] = acc[4 * g + jj] + bias;
      if (which < 2) {
        bf16_t* dst = which == 0 ? ep.q : ep.k;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj) {
          const int row = r0 + jj;
          if (row < M) {
            const int b = row / S;
            const int s = row - b * S;
            dst[((static_cast<int64_t>(b) * ep.num_heads + h) * S + s) * hd + d] = f32_to_bf16(y[jj]);
          }
        }
      } else {
        const int b0 = r0 / S;
        const int s0 = r0 - b0 * S;
        if (r0 + 3 < M && s0 + 3 < S && (ep.ld_vt & 3) == 0 && (s0 & 3) == 0) {
          bf16_t* dst = ep.v_t + ((static_cast<int64_t>(b0) * ep.num_heads + h) * hd + d) * ep.ld_vt + s0;
          *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
        } else {
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int row = r0 + jj;
            if (row < M) {
              const int b = row / S;
              const int s = row - b * S;
              ep.v_t[((static_cast<int64_t>(b) * ep.num_heads + h) * hd + d) * ep.ld_vt + s] = f32_to_bf16(y[jj]);
            }
          }
        }
      }
    }
  } else {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int row = row0 + 8 * (r >> 2) + 4 * lhi + (r & 3);
      if (row < M) store_row_major<EPI>(ep, N, row, col, acc[r], bias);
    }
  }
}

// SPLIT > 1 reproduces the K-split reduction order hipBLASLt picks for some
// small-M shapes: the K range is cut into CW-wide chunks, chunk c is accumulated
// into partial (c % SPLIT) in ascending order, and the partials are added
// left to right before the bias.  All partials live in registers of the same
// wavefront, so the split costs registers, not a second pass.
template <int BM, int BN, int EPI, int SPLIT = 1, int CW = kBK>
__global__ void __launch_bounds__(kThreads)
gemm_bf16_kernel(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W, int M, int N, int K,
                 GemmEpilogueArgs ep) {
  constexpr int RM = BM / 64;  // 32x32 blocks per wavefront along M
  constexpr int RN = BN / 64;  // ... along N
  // K tiles after which the chunk -> partial assignment repeats (even, so the
  // double-buffer index is also a compile-time value inside one period).
  constexpr int PERIOD = (SPLIT == 1) ? 2 : ((CW * SPLIT / kBK) < 2 ? 2 : CW * SPLIT / kBK);
  static_assert(SPLIT == 1 || (CW % 16 == 0 && (CW * SPLIT) % kBK == 0), "bad split chunk");
  constexpr int A_LOADS = BM * (kBK / 8) / kThreads;
  constexpr int B_LOADS = BN * (kBK / 8) / kThreads;
  static_assert(A_LOADS >= 1 && B_LOADS >= 1, "tile too small for 256 threads");

  __shared__ __attribute__((aligned(16))) bf16_t sA[2][BM * kLdk];
  __shared__ __attribute__((aligned(16))) bf16_t sB[2][BN * kLdk];

  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  int tm, tn;
  map_tile(tiles_m, tiles_n, blockIdx.x, &tm, &tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;

  u32x4 ra[A_LOADS];
  u32x4 rb[B_LOADS];

  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int c = tid + i * kThreads;
      const int row = c >> 3;
      const int kc = c & 7;
      const int grow = m0 + row;
      if (grow < M) {
        ra[i] = *reinterpret_cast<const u32x4*>(A + static_cast<int64_t>(grow) * K + k0 + kc * 8);
      } else {
        ra[i] = u32x4{0, 0, 0, 0};
      }
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int c = tid + i * kThreads;
      const int row = c >> 3;
      const int kc = c & 7;
      rb[i] = *reinterpret_cast<const u32x4*>(W + static_cast<int64_t>(n0 + row) * K + k0 + kc * 8);
    }
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(&sA[buf][(c >> 3) * kLdk + (c & 7) * 8]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(&sB[buf][(c >> 3) * kLdk + (c & 7) * 8]) = rb[i];
    }
  };

  f32x16 acc[SPLIT][RM][RN];
#pragma unroll
  for (int p = 0; p < SPLIT; ++p)
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int j = 0; j < RN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[p][i][j][r] = 0.f;

  const int KT = K / kBK;
  load_global(0);
  store_lds(0);
  __syncthreads();

  const int a_base = (wm * (BM / 2) + l32) * kLdk + lhi * 8;
  const int b_base = (wn * (BN / 2) + l32) * kLdk + lhi * 8;

  // KT is a multiple of PERIOD except for SPLIT == 1, where the tail of the
  // last period is skipped by the kt < KT test.
  for (int kt0 = 0; kt0 < KT; kt0 += PERIOD) {
#pragma unroll
    for (int pt = 0; pt < PERIOD; ++pt) {
      const int kt = kt0 + pt;
      if (SPLIT == 1 && kt >= KT) break;
      const int cur = pt & 1;
      if (kt + 1 < KT) load_global((kt + 1) * kBK);
#pragma unroll
      for (int ks = 0; ks < kBK / 16; ++ks) {
        const int part = SPLIT == 1 ? 0 : ((pt * kBK + ks * 16) / CW) % SPLIT;
        bf16x8 af[RM];
        bf16x8 bfr[RN];
#pragma unroll
        for (int i = 0; i < RM; ++i)
          af[i] = *reinterpret_cast<const bf16x8*>(&sA[cur][a_base + i * 32 * kLdk + ks * 16]);
#pragma unroll
        for (int j = 0; j < RN; ++j)
          bfr[j] = *reinterpret_cast<const bf16x8*>(&sB[cur][b_base + j * 32 * kLdk + ks * 16]);
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
          for (int j = 0; j < RN; ++j)
            acc[part][i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], acc[part][i][j], 0, 0, 0);
      }
      if (kt + 1 < KT) store_lds(cur ^ 1);
      __syncthreads();
    }
  }
#pragma unroll
  for (int p = 1; p < SPLIT; ++p)
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int j = 0; j < RN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[0][i][j][r] += acc[p][i][j][r];

  // ---- epilogue ----
  const int row_base = m0 + wm * (BM / 2);
  const int col_base = n0 + wn * (BN / 2);
#pragma unroll
  for (int j = 0; j < RN; ++j) {
#pragma unroll
    for (int i = 0; i < RM; ++i)
      store_block<EPI>(ep, M, N, row_base + i * 32, col_base + j * 32, acc[0][i][j]);
  }
}


// ---------------------------------------------------------------------------
// Narrow-shape kernel, for N or K that is a multiple of 32 but not of 64
// (d_model 32: K = 32, N = 32 or 96).  One wavefront per 32x32 output block;
// the MFMA fragments come straight from global memory (lane (r = l % 32,
// h = l / 32) loads the 16 bytes at K offset 16 ks + 8 h of A row r and of W
// row r) and K accumulates sequentially in 16-deep MFMA steps, the order of
// the unsplit kernels.  At these sizes neither LDS staging nor larger tiles
// pay.
template <int EPI>
__global__ void __launch_bounds__(kThreads)
gemm_narrow_kernel(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W, int M, int N, int K,
                   GemmEpilogueArgs ep) {
  const int lane = threadIdx.x % kWave;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;
  const int blocks_n = N / 32;
  const int64_t blocks = static_cast<int64_t>((M + 31) / 32) * blocks_n;
  const int64_t blk = static_cast<int64_t>(blockIdx.x) * (kThreads / kWave) + threadIdx.x / kWave;
  if (blk >= blocks) return;  // uniform per wavefront; the kernel has no barrier
  const int row0 = static_cast<int>(blk / blocks_n) * 32;
  const int col0 = static_cast<int>(blk % blocks_n) * 32;
  const int arow = min(row0 + l32, M - 1);  // rows past M re-load the last row, never stored
  const bf16_t* a = A + static_cast<int64_t>(arow) * K + lhi * 8;
  const bf16_t* w = W + static_cast<int64_t>(col0 + l32) * K + lhi * 8;
  f32x16 acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = 0.f;
  for (int k0 = 0; k0 < K; k0 += 16) {
    const bf16x8 af = *reinterpret_cast<const bf16x8*>(a + k0);
    const bf16x8 wf = *reinterpret_cast<const bf16x8*>(w + k0);
    acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af, wf, acc, 0, 0, 0);
  }
  store_block<EPI>(ep, M, N, row0, col0, acc);
}

// ---------------------------------------------------------------------------
// Large-tile kernel: BM x BN output tile (256x256, 256x128 or 128x128), four
// wavefronts in a 2 x 2 grid, each owning a (BM/2) x (BN/2) sub-tile of 32x32
// fp32 accumulator blocks (up to 256 registers per lane, held in AGPRs).
//
// Operands move global -> LDS with buffer_load_dwordx4 ... lds, without
// register staging: one instruction writes 64 consecutive 16-byte LDS chunks,
// one per lane, so the LDS layout is chosen on the global side.  An LDS row holds one
// A or W row of the BK-wide K slice as BK/8 chunks of 8 bf16, chunk c stored
// in slot c ^ swz(row) (swz = row & 7 for 8 chunks a row, (row >> 1) & 3 for
// 4), so the 32 rows one MFMA fragment read touches at one K chunk land in
// distinct bank groups.  NS LDS stages form a ring: the loads of K block
// k + NS - 1 are issued while block k is multiplied, and each iteration waits
// only for block k + 1 (s_waitcnt vmcnt with the later blocks' loads still
// outstanding).  The fragments of the next 16-wide K step are read while the
// current step's MFMAs run.
//
// Epilogue: y = bf16(acc + bias) (the nn.Linear output) is staged in LDS as a
// row-major [BM][BN+8] bf16 tile, then every thread finishes 8 consecutive
// outputs of one row (GELU / residual / row mask), so the residual reads and
// the output writes are 16-byte coalesced; the QKV epilogue writes Q and K
// rows of 8 head channels and V^T columns of 8 sequence positions.
constexpr int kLdsLimitBytes = 160 * 1024;


template <int BM, int BN, int BK, int NS>
struct BigTile {
  static constexpr int kRM = BM / 64;                       // 32x32 blocks per wave along M
  static constexpr int kRN = BN / 64;                       // ... along N
  static constexpr int kStage = (BM + BN) * BK;             // bf16 elements per LDS stage
  static constexpr int kChunks = BK / 8;                    // 16-byte chunks per LDS row
  static constexpr int kRowsPerLoad = kWave / kChunks;      // rows one load instruction fills
  static constexpr int kLoadsA = BM / (4 * kRowsPerLoad);   // per thread per stage
  static constexpr int kLoadsB = BN / (4 * kRowsPerLoad);
  static constexpr int kLoads = kLoadsA + kLoadsB;
  static constexpr int kLdc = BN + 8;                       // epilogue tile row stride
  static constexpr int kSmem = (NS * kStage > BM * kLdc) ? NS * kStage : BM * kLdc;
  static_assert(BK == 32 || BK == 64, "BK");
  static_assert(kSmem * 2 <= kLdsLimitBytes, "LDS budget");
  static_assert(NS >= 2 && kLoads * (NS - 2) < 64, "vmcnt range");
  __device__ static constexpr int swz(int row) { return kChunks == 8 ? (row & 7) : ((row >> 1) & 3); }
};

// v: 8 consecutive outputs y = bf16(acc + bias) of one row, two per word
// (low half first).  r / keep: the residual's 8 values and the row-mask
// verdict, loaded ahead by the caller (residual epilogues only).
template <int EPI>
__device__ __forceinline__ void finish8(const GemmEpilogueArgs& ep, int N, int row, int col, u32x4 v,
                                        u32x4 r = u32x4{0u, 0u, 0u, 0u}, bool keep = true,
                                        bool gelu_table = false, const bf16_t* gelu_tab = nullptr) {
  const int64_t idx = static_cast<int64_t>(row) * N + col;
  u32x4 w;
  if constexpr (EPI == kEpiBias) {
    w = v;
  } else if constexpr (EPI == kEpiBiasGelu) {
    if (gelu_table) {
      // the compact table in LDS (gelu8_lds) gives the erf GELU of each value
      w = gelu8_lds(gelu_tab, v);
    } else {
      float g[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        g[2 * e] = gelu_erf(lo_bf16(v[e]));
        g[2 * e + 1] = gelu_erf(hi_bf16(v[e]));
      }
      w = u32x4{pack_bf16x2(g[0], g[1]), pack_bf16x2(g[2], g[3]), pack_bf16x2(g[4], g[5]), pack_bf16x2(g[6], g[7])};
    }
  } else {
    if (keep) {
      float o[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        o[2 * e] = lo_bf16(r[e]) + lo_bf16(v[e]);
        o[2 * e + 1] = hi_bf16(r[e]) + hi_bf16(v[e]);
      }
      w = u32x4{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3]), pack_bf16x2(o[4], o[5]), pack_bf16x2(o[6], o[7])};
    } else {
      w = (EPI == kEpiResidualKeep) ? r : u32x4{0u, 0u, 0u, 0u};
    }
  }
  *reinterpret_cast<u32x4*>(ep.out + idx) = w;
}

template <int BM, int BN, int BK, int NS, int EPI, int OCC = 1>
__global__ void __launch_bounds__(kThreads, OCC)
gemm_big_kernel(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W, int M, int N, int K,
                GemmEpilogueArgs ep) {
  using T = BigTile<BM, BN, BK, NS>;
  constexpr int RM = T::kRM, RN = T::kRN;
  // GELU products append the compact GELU table (2 kGeluSpan entries) and one
  // word for the workgroup's table verdict
  constexpr int kGeluLds = EPI == kEpiBiasGelu ? 2 * kGeluSpan + 2 : 0;
  static_assert((T::kSmem + kGeluLds) * 2 * OCC <= kLdsLimitBytes, "LDS budget for OCC workgroups per CU");
  __shared__ __attribute__((aligned(16))) bf16_t smem[T::kSmem + kGeluLds];

  const int tiles_m = (M + BM - 1) / BM;
  const int tiles_n = N / BN;
  int tm, tn;
  map_tile(tiles_m, tiles_n, blockIdx.x, &tm, &tn);
  const int m0 = tm * BM;
  const int n0 = tn * BN;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;
  // The GELU table's ready flag, read by wavefront 0 now (an agent-scope
  // atomic load, so it sees the value in memory rather than a cached copy)
  // and handed to the workgroup through LDS at the last K block's barrier:
  // one verdict per workgroup, taken before any table word is read.  A clear flag
  // (a product on another stream racing the first fill) selects the erf.
  uint32_t gelu_flag = 0u;
  if constexpr (EPI == kEpiBiasGelu) {
    if (wave == 0) gelu_flag = __hip_atomic_load(&g_gelu_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }

  // Load instruction j of wavefront w fills LDS rows R (4 j + w) .. + R - 1
  // (R = rows per instruction); lane -> row + lane / chunks, slot lane % chunks,
  // holding global chunk slot ^ swz(row).  Offsets are relative to the tile's
  // first row (32-bit); the bases are uniform.
  const int lrow = lane / T::kChunks;
  const int gcol = ((lane % T::kChunks) ^ T::swz(lrow)) * 8;
  // Each load instruction reads [tile base + uniform K offset + per-lane 32-bit
  // byte offset]; the per-lane offsets do not change along K (the compiler
  // hoists them).  (They are not precomputed into an array: a local array
  // captured by the loading lambda makes clang's host pass drop the kernel's
  // launch stub.)
  const char* a_tile = reinterpret_cast<const char*>(A + static_cast<int64_t>(m0) * K);
  const int a_rows_left = M - 1 - m0;  // rows past M re-load the last row, never stored
  // W comes from nn.Linear's [N, K] layout (row stride K) or from the
  // tile-packed copy [N / PN][K / 32][PN][32] (gemm_prepack_weight), where the
  // tile's rows of one 32-deep K slice are contiguous: row r, column c of
  // stage k0 sits at group base + k0 * PN + (c / 32) * PN * 32 + (n0 % PN + r)
  // * 32 + c % 32 elements.  Same values in the same LDS slots either way.
  const bool w_packed = ep.w_packed != nullptr;
  const int pn = ep.w_packed_rows;
  const char* w_tile = w_packed ? reinterpret_cast<const char*>(ep.w_packed + static_cast<int64_t>(n0 - n0 % pn) * K)
                                : reinterpret_cast<const char*>(W + static_cast<int64_t>(n0) * K);
  const int w_k_mul = w_packed ? pn : 1;  // element step of W per unit of k0
  // The ring loads are buffer loads on per-tile resources: a lane's operand is
  // a 32-bit offset (hoisted out of the K loop) and the K step a uniform
  // soffset.  With 64-bit per-lane addresses (global_load_lds) the same loads
  // took more issue time away from the MFMAs: 1-4% slower on every wide
  // product, same bits.
  const i32x4 a_rsrc = buffer_rsrc(a_tile);
  const i32x4 w_rsrc = buffer_rsrc(w_tile);
  const int w_row0 = w_packed ? n0 % pn : 0;

  // kM16 (the four-stage ring of 32-deep blocks): v_mfma_f32_16x16x32_bf16
  // on 16x16 blocks, one MFMA per block and K block; otherwise
  // v_mfma_f32_32x32x16_bf16 on 32x32 blocks, two 16-deep steps per 32 of K.
  // On MI355X the two forms give bitwise the same outputs (both match
  // torch's products on every tested shape); the 16x16x32 form moves half
  // the accumulator registers per product, and under the power cap its
  // launches run at a higher shader clock.
  constexpr bool kM16 = BK == 32 && NS == 4 && BM == 256 && BN == 256 && EPI != kEpiBiasGelu;
  constexpr int FM = kM16 ? BM / 32 : RM;  // fragments per wavefront along M (16 or 32 rows each)
  constexpr int FN = kM16 ? BN / 32 : RN;  // ... along N
  constexpr int kFR = kM16 ? 16 : 32;      // rows per fragment
  f32x16 acc[kM16 ? 1 : RM][kM16 ? 1 : RN];
  f32x4 acc4[kM16 ? FM : 1][kM16 ? FN : 1];
  if constexpr (kM16) {
#pragma unroll
    for (int i = 0; i < FM; ++i)
#pragma unroll
      for (int j = 0; j < FN; ++j) acc4[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  } else {
#pragma unroll
    for (int i = 0; i < RM; ++i)
#pragma unroll
      for (int j = 0; j < RN; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.f;
  }

  // Fragment rows: A row wm*(BM/2) + kFR i + fr, W row wn*(BN/2) + kFR j + fr
  // (fr = the lane's row in the fragment); the row's low bits are fr's, so the
  // swizzle is per lane.  A lane reads 8 consecutive k: chunk fk of the step.
  const int fr = kM16 ? lane % 16 : l32;
  const int fk = kM16 ? lane / 16 : lhi;
  const int a_off = (wm * (BM / 2) + fr) * BK;
  const int b_off = BM * BK + (wn * (BN / 2) + fr) * BK;
  const int swz = T::swz(fr);
  auto read_frags = [&](int stage, int ks, bf16x8 (&af)[FM], bf16x8 (&bf)[FN]) {
    const bf16_t* st = smem + stage * T::kStage;
    const int slot = ((kM16 ? fk : 2 * ks + fk) ^ swz) * 8;
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const bf16x8*>(st + a_off + i * kFR * BK + slot);
#pragma unroll
    for (int j = 0; j < FN; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(st + b_off + j * kFR * BK + slot);
  };
  constexpr int KS = kM16 ? 1 : BK / 16;  // MFMA steps per block
  // A block's loads go out in KS parts, one per step.  With more than two
  // stages, block kt + NS - 1's parts go out over block kt's steps.  With two
  // stages (NS == 2) block kt + 1's loads must all be requested before block
  // kt's barrier, so its part 0 goes out in block kt - 1's last step (after
  // that block's barrier, when the stage it read is free) and parts 1 .. KS-1
  // over block kt's first KS - 1 steps.
  constexpr int kPer = T::kLoads / KS;  // load instructions issued per step
  static_assert(T::kLoads % KS == 0, "a block's loads split evenly over its steps");
  // Part `part` of a block's loads: instructions [part * kPer, (part + 1) * kPer)
  // of the list (A rows, then W rows).
  // (The global loads are written out here rather than in helper lambdas: a
  // device builtin in a lambda called from another lambda makes clang's host
  // pass drop the kernel's launch stub.)
  auto issue_part = [&](int stage, int k0, int part) {
    bf16_t* sa = smem + stage * T::kStage;
#pragma unroll
    for (int q = 0; q < T::kLoads; ++q) {
      if (q < part * kPer || q >= (part + 1) * kPer || q >= T::kLoads) continue;
      const bool is_a = q < T::kLoadsA;
      const int row = T::kRowsPerLoad * (4 * (is_a ? q : q - T::kLoadsA) + wave);
      const uint32_t off =
          is_a ? static_cast<uint32_t>(min(row + lrow, a_rows_left) * K + gcol) * 2u
          : w_packed ? static_cast<uint32_t>((gcol >> 5) * pn * 32 + (w_row0 + row + lrow) * 32 + (gcol & 31)) * 2u
                     : static_cast<uint32_t>((row + lrow) * K + gcol) * 2u;
      enc_buffer_load_lds(is_a ? a_rsrc : w_rsrc,
                      reinterpret_cast<__attribute__((address_space(3))) uint32_t*>(
                          reinterpret_cast<uintptr_t>(sa + (is_a ? 0 : BM * BK) + row * BK)),
                      16, static_cast<int>(off), is_a ? 2 * k0 : 2 * k0 * w_k_mul, 0, 0);
    }
  };
  // Wait until at most n of this thread's load instructions are in flight and
  // its LDS reads are done (n is one of the counts the K loop uses; anything
  // else waits for everything).
  constexpr int kSteadyLater = NS == 2 ? 0 : (NS - 2) * T::kLoads - kPer;
  static_assert(NS >= 2 && NS <= 4 && kSteadyLater >= 0 && 2 * T::kLoads < 64, "vmcnt range");
  auto wait_vm = [&](int n) {
    if (n == kSteadyLater) {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(kSteadyLater, 0));
    } else if (n == T::kLoads) {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(T::kLoads, 0));
    } else if (n == 2 * T::kLoads) {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(2 * T::kLoads, 0));
    } else if (n == kPer) {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(kPer, 0));
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    }
  };
  // The W fragment is the MFMA's A operand and the A fragment its B operand,
  // so block (i, j) accumulates the transposed product: lane l32 holds output
  // row wm*(BM/2) + 32 i + l32 and register r output column
  // wn*(BN/2) + 32 j + 8 (r / 4) + 4 lhi + r % 4 -- runs of four consecutive
  // columns per lane, which the epilogue stages with one 8-byte LDS write
  // instead of four 2-byte ones.  Each output is the same 16-term dot
  // products summed into the same chain as in the untransposed order, so the
  // values are the same bit for bit.  (Each library timed alone in its own
  // process: 1-3% faster on every wide tile.)
  //
  // One K step: MFMA q (block q / RN, q % RN) with fragment read q of the
  // next step and load q of the step's part of the ring loads next to it,
  // each group closed by a scheduling barrier, so the reads and loads go out
  // one per MFMA while the matrix pipe is busy.  With `sched_group_barrier`
  // hints for the same pattern the scheduler still bunched up to five loads
  // and seven reads between two MFMAs, which the one wavefront per SIMD
  // issues in order while its MFMA pipe idles: the fixed order is 2-5%
  // faster on the wide products, bitwise the same.
  auto step_explicit = [&](const bf16x8 (&a)[FM], const bf16x8 (&b)[FN], bf16x8 (&an)[FM], bf16x8 (&bn)[FN],
                           int rstage, int rks, bool read, int lstage, int lk0, int part, bool load)
      __attribute__((always_inline)) {
    const bf16_t* rs = smem + rstage * T::kStage;
    const int slot = ((2 * rks + lhi) ^ swz) * 8;
    bf16_t* sa = smem + lstage * T::kStage;
#pragma unroll
    for (int q = 0; q < RM * RN; ++q) {
      const int i = q / RN, j = q % RN;
      if constexpr (!kM16) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(b[j], a[i], acc[i][j], 0, 0, 0);
      if (read && q < RM) an[q] = *reinterpret_cast<const bf16x8*>(rs + a_off + q * 32 * BK + slot);
      if (read && q >= RM && q < RM + RN)
        bn[q - RM] = *reinterpret_cast<const bf16x8*>(rs + b_off + (q - RM) * 32 * BK + slot);
      // With four stages (the tile-packed weight's ring) the loads go after the
      // reads (1-2% faster there); the two-stage ring keeps them beside the
      // reads (its loads must all be out before the block's barrier).
      constexpr int kLoadAt = (NS > 2 && RM + RN + kPer <= RM * RN) ? RM + RN : 0;
      const int lq = part * kPer + (q - kLoadAt);
      if (load && q >= kLoadAt && q - kLoadAt < kPer && lq < T::kLoads) {
        const bool is_a = lq < T::kLoadsA;
        const int row = T::kRowsPerLoad * (4 * (is_a ? lq : lq - T::kLoadsA) + wave);
        const uint32_t off =
            is_a ? static_cast<uint32_t>(min(row + lrow, a_rows_left) * K + gcol) * 2u
            : w_packed ? static_cast<uint32_t>((gcol >> 5) * pn * 32 + (w_row0 + row + lrow) * 32 + (gcol & 31)) * 2u
                       : static_cast<uint32_t>((row + lrow) * K + gcol) * 2u;
        enc_buffer_load_lds(is_a ? a_rsrc : w_rsrc,
                            reinterpret_cast<__attribute__((address_space(3))) uint32_t*>(
                                reinterpret_cast<uintptr_t>(sa + (is_a ? 0 : BM * BK) + row * BK)),
                            16, static_cast<int>(off), is_a ? 2 * lk0 : 2 * lk0 * w_k_mul, 0, 0);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };

  // Prologue: blocks 0 .. NS-2 in full; block NS-1 loads during block 0
  // (two stages: block 1's part 0 goes out here, after block 0's loads).
  const int KT = K / BK;
  // (kM16: always NS - 1 blocks, past the last block re-reading it into a
  // stage nobody reads, so that every block's wait is the same)
  const int prologue = kM16 ? NS - 1 : min(NS - 1, KT);
  for (int p = 0; p < prologue; ++p)
#pragma unroll
    for (int part = 0; part < KS; ++part) issue_part(p, min(p, KT - 1) * BK, part);
  if (NS == 2 && KT > 1) {
    issue_part(1, BK, 0);
    wait_vm(kPer);
  } else {
    wait_vm((prologue - 1) * T::kLoads);
  }
  ring_barrier();
  bf16x8 af[FM], bf[FN];
  if constexpr (kM16) {
    // block 0's W fragments 0..3, then its A fragments: the order in which
    // each block reads the next one's, so that the compiler's LDS waits at
    // the top of the K loop are the same from the loop's entry and its back
    // edge (W fragments 4..7 are read inside the block)
    const int slot = (fk ^ swz) * 8;
#pragma unroll
    for (int j = 0; j < FN / 2; ++j) bf[j] = *reinterpret_cast<const bf16x8*>(smem + b_off + j * kFR * BK + slot);
#pragma unroll
    for (int i = 0; i < FM; ++i) af[i] = *reinterpret_cast<const bf16x8*>(smem + a_off + i * kFR * BK + slot);
  } else {
    read_frags(0, 0, af, bf);
  }

  // K block kt (in LDS stage `stage`).  Every step multiplies while the next
  // step's fragments are read and one part of a later block's loads is
  // requested into a free stage, so the loads are spread over the block
  // instead of bunched.  Before the last step comes the one barrier:
  // block kt + 1 has landed for every wavefront and nobody reads stage `stage`
  // any more; the last step then reads step 0 of block kt + 1, so no LDS or
  // memory latency is left exposed between blocks.  `load` covers the parts
  // issued before the barrier, `load_last` the last step's part (two stages:
  // part 0 of block kt + 2, into stage `stage`).
  // (A plain lambda called with constant flags: a generic lambda makes clang
  // drop the kernel's host-side launch stub, and runtime flags would merge
  // differently scheduled MFMA results and double the accumulator registers.)
  auto k_block = [&](int kt, int stage, int later, bool load, bool next, bool load_last)
      __attribute__((always_inline)) {
    const int lstage = stage == 0 ? NS - 1 : stage - 1;  // stage of block kt + NS - 1
    const int lk0 = (kt + NS - 1) * BK;
    constexpr int kPart0 = NS == 2 ? 1 : 0;  // part of the first step
#pragma unroll
    for (int ks = 0; ks + 1 < KS; ++ks) {
      bf16x8 an[FM], bn[FN];
      step_explicit(af, bf, an, bn, stage, ks + 1, true, lstage, lk0, ks + kPart0, load);
#pragma unroll
      for (int i = 0; i < RM; ++i) af[i] = an[i];
#pragma unroll
      for (int j = 0; j < RN; ++j) bf[j] = bn[j];
    }
    if constexpr (EPI == kEpiBiasGelu) {
      // last block: every load has to land before this barrier anyway, so
      // wavefront 0 publishes its flag reading here at no cost, in the slot
      // after the compact table (outside the ring and the staging area)
      if (!next && tid == 0) reinterpret_cast<uint32_t*>(smem + T::kSmem)[kGeluSpan] = gelu_flag;
    }
    wait_vm(next ? later : 0);  // loads requested after block kt + 1; the epilogue reuses the ring
    ring_barrier();
    bf16x8 an[FM], bn[FN];
    if constexpr (NS == 2)
      step_explicit(af, bf, an, bn, stage + 1 == NS ? 0 : stage + 1, 0, next, stage, lk0 + BK, 0, load_last);
    else
      step_explicit(af, bf, an, bn, stage + 1 == NS ? 0 : stage + 1, 0, next, lstage, lk0, KS - 1, load_last);
    if (next) {
#pragma unroll
      for (int i = 0; i < RM; ++i) af[i] = an[i];
#pragma unroll
      for (int j = 0; j < RN; ++j) bf[j] = bn[j];
    }
  };
  int stage = 0;
  int kt = 0;
  if constexpr (kM16) {
    // One 32-deep block, one step: after the wait for block kt + 1 and the
    // barrier, its 64 MFMAs in two halves (W fragments j = 0..3, then 4..7,
    // A fragments i-major inside each).  The fragments are read in place,
    // each after its last use, so there is one register set and no copies:
    // this block's W fragments 4..7 over the first half; the next block's W
    // fragments 0..3 (last used in the first half) and A fragment i (after
    // its last MFMA) over the second.  Loads go out one per eight MFMAs, for
    // block kt + 3 (clamped to the last block).
    auto step16 = [&](int cstage, int nstage, bool next, int lstage, int lk0, bool load)
        __attribute__((always_inline)) {
      const bf16_t* cs = smem + cstage * T::kStage;
      const bf16_t* ns = smem + nstage * T::kStage;
      const int slot = (fk ^ swz) * 8;
      bf16_t* sa = smem + lstage * T::kStage;
#pragma unroll
      for (int q = 0; q < FM * FN; ++q) {
        const int h = q / (FM * FN / 2), i = (q % (FM * FN / 2)) / (FN / 2), j = (FN / 2) * h + q % (FN / 2);
        acc4[i][j] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(bf[j], af[i], acc4[i][j], 0, 0, 0);
        if (q < FN / 2)
          bf[FN / 2 + q] = *reinterpret_cast<const bf16x8*>(cs + b_off + (FN / 2 + q) * kFR * BK + slot);
        if (next && h == 1 && q - FM * FN / 2 < FN / 2)
          bf[q - FM * FN / 2] = *reinterpret_cast<const bf16x8*>(ns + b_off + (q - FM * FN / 2) * kFR * BK + slot);
        if (next && h == 1 && q % (FN / 2) == FN / 2 - 1)
          af[i] = *reinterpret_cast<const bf16x8*>(ns + a_off + i * kFR * BK + slot);
        constexpr int kLS = (FM * FN) / kPer;
        if (load && q % kLS == kLS / 2) {
          const int lq = q / kLS;
          const bool is_a = lq < T::kLoadsA;
          const int row = T::kRowsPerLoad * (4 * (is_a ? lq : lq - T::kLoadsA) + wave);
          const uint32_t off =
              is_a ? static_cast<uint32_t>(min(row + lrow, a_rows_left) * K + gcol) * 2u
              : w_packed ? static_cast<uint32_t>((gcol >> 5) * pn * 32 + (w_row0 + row + lrow) * 32 + (gcol & 31)) * 2u
                         : static_cast<uint32_t>((row + lrow) * K + gcol) * 2u;
          enc_buffer_load_lds(is_a ? a_rsrc : w_rsrc,
                              reinterpret_cast<__attribute__((address_space(3))) uint32_t*>(
                                  reinterpret_cast<uintptr_t>(sa + (is_a ? 0 : BM * BK) + row * BK)),
                              16, static_cast<int>(off), is_a ? 2 * lk0 : 2 * lk0 * w_k_mul, 0, 0);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    };
    for (; kt + 1 < KT; ++kt) {
      const int nstage = stage + 1 == NS ? 0 : stage + 1;
      // block kt + 1 has landed; block kt + 2's loads may be in flight, and so
      // may the read of block kt + 1's last A fragment (its stage is not
      // written before block kt + 2's barrier)
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(kSteadyLater, 15));
      ring_barrier();
      step16(stage, nstage, true, stage == 0 ? NS - 1 : stage - 1, min(kt + NS - 1, KT - 1) * BK, true);
      stage = nstage;
    }
    wait_vm(0);
    ring_barrier();
    step16(stage, stage, false, stage, 0, false);
    ring_barrier();  // this block's last fragment reads are done before the epilogue reuses the ring
  } else if constexpr (NS == 2) {
    // every load in flight at a block's barrier is for the next block
    for (; kt + 2 < KT; ++kt) {
      k_block(kt, stage, 0, true, true, true);
      stage ^= 1;
    }
    if (kt + 1 < KT) {
      k_block(kt, stage, 0, true, true, false);
      stage ^= 1;
      ++kt;
    }
  } else {
    for (; kt + NS - 1 < KT; ++kt) {
      k_block(kt, stage, kSteadyLater, true, true, true);
      stage = stage + 1 == NS ? 0 : stage + 1;
    }
    for (; kt + 1 < KT; ++kt) {
      k_block(kt, stage, (KT - 2 - kt) * T::kLoads, false, true, false);
      stage = stage + 1 == NS ? 0 : stage + 1;
    }
  }
  if constexpr (!kM16) k_block(kt, stage, 0, false, false, false);

  // ---- epilogue: y = bf16(acc + bias) into LDS, then 8 outputs per thread ----
  constexpr int kPerRow = BN / 8;
  constexpr int kRowsPerPass = kThreads / kPerRow;
  constexpr int kPasses = BM / kRowsPerPass;
  constexpr bool kResidual = EPI == kEpiResidualKeep || EPI == kEpiResidualZero;
  const int c8 = (tid % kPerRow) * 8;
  const int rl0 = tid / kPerRow;
  // The residual rows (and row-mask bytes) of the first kDepth passes are
  // requested before the outputs are read back, and pass p requests pass
  // p + kDepth, so the memory latency overlaps the staging and the passes
  // instead of costing one round trip per pass.  Rows past M read row M-1 and
  // are never stored.
  constexpr int kDepth = kPasses < 2048 / BN ? kPasses : 2048 / BN;  // 16 or 8: within the register budget
  u32x4 res[kResidual ? kDepth : 1];
  // The mask bytes are held untested until their pass: a test here would
  // wait for the byte's load, and with it for every load requested before
  // it.  Without a mask the loads read the residual's first byte (any valid
  // address), which the pass ignores.
  uint32_t keep[kResidual ? kDepth : 1];
  const bool has_mask = ep.row_mask != nullptr;
  const uint8_t* mask_bytes = has_mask ? ep.row_mask : reinterpret_cast<const uint8_t*>(ep.residual);
  auto load_residual = [&](int p, u32x4& r, uint32_t& k) {
    const int row = min(m0 + rl0 + p * kRowsPerPass, M - 1);
    r = *reinterpret_cast<const u32x4*>(ep.residual + static_cast<int64_t>(row) * N + n0 + c8);
    k = mask_bytes[has_mask ? row : 0];
  };
  // (256-wide tiles: requested after the staging, which needs the registers)
  if constexpr (kResidual && BN <= 128) {
#pragma unroll
    for (int p = 0; p < kDepth; ++p) load_residual(p, res[p], keep[p]);
  }
  bf16_t* sc = smem;  // every wave passed the last barrier: the stages are free
  // GELU: the workgroup's verdict (wavefront 0's reading of the ready flag,
  // in LDS since the last K block's barrier).  With the table, its compact words are
  // requested now, so their latency overlaps the staging below, and written
  // to LDS before the staging barrier.  No table word is read before a flag
  // reading of 1, and the flag is set on the fill's stream after the fill
  // kernel ended (its writes are in memory by then), so no cache can hold a
  // word from before the fill; with a clear flag the words are never read.
  bf16_t* gelu_tab = smem + T::kSmem;
  constexpr int kGeluWords = kGeluSpan;  // 4-byte words of both slices
  constexpr int kGeluWordsPerThread = (kGeluWords + kThreads - 1) / kThreads;
  const bool table =
      EPI == kEpiBiasGelu && __builtin_amdgcn_readfirstlane(reinterpret_cast<const uint32_t*>(gelu_tab)[kGeluWords]) != 0;
  uint32_t gelu_words[EPI == kEpiBiasGelu ? kGeluWordsPerThread : 1];
  if constexpr (EPI == kEpiBiasGelu) {
    if (table) {
#pragma unroll
      for (int i = 0; i < kGeluWordsPerThread; ++i) {
        const int w = tid + i * kThreads;  // word w of the LDS table
        const int half_words = kGeluSpan / 2;
        const uint32_t src = (w < half_words ? kGeluLo : 0x8000u + kGeluLo) + 2u * (w % half_words);
        if (w < kGeluWords) gelu_words[i] = *reinterpret_cast<const uint32_t*>(&g_gelu_table[src]);
      }
    }
  }
  if constexpr (kM16) {
    // 16x16 blocks: lane l holds row (token) l % 16 and the four consecutive
    // columns 4 (l / 16) .. + 3 of block (i, j)
#pragma unroll
    for (int j = 0; j < FN; ++j) {
      const int cl = wn * (BN / 2) + j * 16 + 4 * fk;  // four consecutive columns
      const u32x2 bb = *reinterpret_cast<const u32x2*>(ep.bias + n0 + cl);
      const float b0 = lo_bf16(bb[0]), b1 = hi_bf16(bb[0]), b2 = lo_bf16(bb[1]), b3 = hi_bf16(bb[1]);
#pragma unroll
      for (int i = 0; i < FM; ++i) {
        const int rl = wm * (BM / 2) + i * 16 + fr;
        *reinterpret_cast<u32x2*>(sc + rl * T::kLdc + cl) =
            u32x2{pack_bf16x2(acc4[i][j][0] + b0, acc4[i][j][1] + b1), pack_bf16x2(acc4[i][j][2] + b2, acc4[i][j][3] + b3)};
      }
    }
  } else {
#pragma unroll
    for (int j = 0; j < RN; ++j) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int cl = wn * (BN / 2) + j * 32 + 8 * g + 4 * lhi;  // four consecutive columns
        const u32x2 bb = *reinterpret_cast<const u32x2*>(ep.bias + n0 + cl);
        const float b0 = lo_bf16(bb[0]), b1 = hi_bf16(bb[0]), b2 = lo_bf16(bb[1]), b3 = hi_bf16(bb[1]);
#pragma unroll
        for (int i = 0; i < RM; ++i) {
          const int rl = wm * (BM / 2) + i * 32 + l32;
          *reinterpret_cast<u32x2*>(sc + rl * T::kLdc + cl) =
              u32x2{pack_bf16x2(acc[i][j][4 * g] + b0, acc[i][j][4 * g + 1] + b1),
                    pack_bf16x2(acc[i][j][4 * g + 2] + b2, acc[i][j][4 * g + 3] + b3)};
        }
      }
    }
  }
  if constexpr (kResidual && BN > 128) {
#pragma unroll
    for (int p = 0; p < kDepth; ++p) load_residual(p, res[p], keep[p]);
  }
  if constexpr (EPI == kEpiBiasGelu) {
    if (table) {
#pragma unroll
      for (int i = 0; i < kGeluWordsPerThread; ++i) {
        const int w = tid + i * kThreads;
        if (w < kGeluWords) reinterpret_cast<uint32_t*>(gelu_tab)[w] = gelu_words[i];
      }
    }
  }
  __syncthreads();
  // Every row of the tile is in range (all tiles but the last tile row): the
  // passes then run without a per-row branch, so the compiler can batch their
  // LDS reads and stores.  Uniform.
  const bool full = m0 + BM <= M;

  if constexpr (EPI != kEpiQkvHeadMajor) {
    // the passes, with the GELU's table (or erf) and the range check fixed
    // for the whole loop
    auto passes = [&](bool gelu_table, bool all_rows) __attribute__((always_inline)) {
#pragma unroll
      for (int p = 0; p < kPasses; ++p) {
        const int rl = rl0 + p * kRowsPerPass;
        const int row = m0 + rl;
        if (all_rows || row < M) {
          const u32x4 v = *reinterpret_cast<const u32x4*>(sc + rl * T::kLdc + c8);
          if constexpr (kResidual) {
            finish8<EPI>(ep, N, row, n0 + c8, v, res[p % kDepth], !has_mask || keep[p % kDepth] != 0u);
          } else {
            finish8<EPI>(ep, N, row, n0 + c8, v, u32x4{0u, 0u, 0u, 0u}, true, gelu_table, gelu_tab);
          }
        }
        if constexpr (kResidual) {
          if (p + kDepth < kPasses) load_residual(p + kDepth, res[p % kDepth], keep[p % kDepth]);
        }
      }
    };
    // One verdict per workgroup (above).  The GELU keeps the per-row branch
    // on full tiles too (batched without it, the table's global gathers this
    // epilogue used before the LDS table ran 1-3% slower).
    if (table) {
      passes(true, false);
    } else if (EPI != kEpiBiasGelu && full) {
      passes(false, true);
    } else {
      passes(false, false);
    }
  } else {
    const int D = ep.d_model;
    const int hd = ep.head_dim;
    const int S = ep.seq_len;
    // Row m0 + rl of the tile is sequence position s of batch b.  On a full
    // tile whose row stride is at most S both loops below carry s and the
    // element offset along (one wrap into the next sequence per step at
    // most); otherwise each row divides.
    auto locate = [&](int row, int& b, int& s) {
      b = row / S;
      s = row - b * S;
    };
    // Q / K: 8 consecutive channels of one head, one row; the thread's
    // channels are the same in every pass.  Element offset of (b, s):
    // ((b H + h) S + s) hd + d.
    const int col = n0 + c8;
    const int which = col / D;
    if (which < 2) {
      const int h = (col - which * D) / hd;
      const int d = (col - which * D) - h * hd;
      bf16_t* dst = which == 0 ? ep.q : ep.k;
      auto offset = [&](int b, int s) {
        return ((static_cast<int64_t>(b) * ep.num_heads + h) * S + s) * hd + d;
      };
      if (full && kRowsPerPass <= S) {
        int b, s;
        locate(m0 + rl0, b, s);
        int64_t off = offset(b, s);
        const int64_t wrap_off = (static_cast<int64_t>(ep.num_heads) - 1) * S * hd;  // next batch, s - S
#pragma unroll
        for (int p = 0; p < kPasses; ++p) {
          *reinterpret_cast<u32x4*>(dst + off) =
              *reinterpret_cast<const u32x4*>(sc + (rl0 + p * kRowsPerPass) * T::kLdc + c8);
          s += kRowsPerPass;
          off += kRowsPerPass * hd;
          const bool wrap = s >= S;
          s = wrap ? s - S : s;
          off = wrap ? off + wrap_off : off;
        }
      } else {
        for (int rl = rl0; rl < BM; rl += kRowsPerPass) {
          const int row = m0 + rl;
          if (row >= M) break;
          int b, s;
          locate(row, b, s);
          *reinterpret_cast<u32x4*>(dst + offset(b, s)) = *reinterpret_cast<const u32x4*>(sc + rl * T::kLdc + c8);
        }
      }
    }
    // V^T on full tiles: two adjacent channels (one head: hd is even), 8
    // consecutive rows (sequence positions).  Thread t owns channels
    // 2 (t % (BN/2)) and +1, and row groups t / (BN/2), + kVStep2, ... of 8
    // rows each: one 4-byte LDS read per row gives both channels' values,
    // and byte permutes split them into one 16-byte V^T store per channel
    // (half the LDS reads of one channel per thread).  Element offset of
    // (b, s): b H hd ld + (h hd + d) ld + s.
    constexpr int kVPairs = BN / 2;
    static_assert(kThreads % kVPairs == 0 && BM % (8 * (kThreads / kVPairs)) == 0, "channel pairs per thread");
    constexpr int kVStep2 = kThreads / kVPairs;
    const int cp = 2 * (tid % kVPairs);
    const bool v_fast = full && (S & 7) == 0 && (ep.ld_vt & 7) == 0 && 8 * kVStep2 <= S;
    if (v_fast && (n0 + cp) / D == 2) {
      const int h = (n0 + cp - 2 * D) / hd;
      const int d = (n0 + cp - 2 * D) - h * hd;
      bf16_t* vrow = ep.v_t + (static_cast<int64_t>(h) * hd + d) * ep.ld_vt;
      const int64_t batch_stride = static_cast<int64_t>(ep.num_heads) * hd * ep.ld_vt;
      int b, s;
      locate(m0 + (tid / kVPairs) * 8, b, s);
      int64_t off = b * batch_stride + s;
#pragma unroll
      for (int it = 0; it < BM / (8 * kVStep2); ++it) {
        const int r8 = (tid / kVPairs + it * kVStep2) * 8;
        uint32_t w[8];  // row r8 + e: channel cp in the low half, cp + 1 in the high half
#pragma unroll
        for (int e = 0; e < 8; ++e) w[e] = *reinterpret_cast<const uint32_t*>(sc + (r8 + e) * T::kLdc + cp);
        u32x4 lo, hi;
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          lo[e] = __builtin_amdgcn_perm(w[2 * e + 1], w[2 * e], 0x05040100u);  // rows 2e, 2e+1 of channel cp
          hi[e] = __builtin_amdgcn_perm(w[2 * e + 1], w[2 * e], 0x07060302u);  // ... of channel cp + 1
        }
        *reinterpret_cast<u32x4*>(vrow + off) = lo;
        *reinterpret_cast<u32x4*>(vrow + ep.ld_vt + off) = hi;
        s += 8 * kVStep2;
        off += 8 * kVStep2;
        const bool wrap = s >= S;
        s = wrap ? s - S : s;
        off = wrap ? off + batch_stride - S : off;
      }
    }
    // V^T otherwise: one channel, 8 consecutive rows.  Thread t owns channel
    // t % BN of the tile and row groups t / BN, t / BN + kVStep, ... of 8 rows
    // each.
    static_assert(kThreads % BN == 0, "one channel per thread");
    constexpr int kVStep = kThreads / BN;
    const int cl = tid % BN;
    const int vcol = n0 + cl;
    if (!v_fast && vcol / D == 2) {
      const int h = (vcol - 2 * D) / hd;
      const int d = (vcol - 2 * D) - h * hd;
      bf16_t* vrow = ep.v_t + (static_cast<int64_t>(h) * hd + d) * ep.ld_vt;
      const int64_t batch_stride = static_cast<int64_t>(ep.num_heads) * hd * ep.ld_vt;
      // 8-row groups that never straddle a sequence and land 16-byte aligned
      if (full && (S & 7) == 0 && (ep.ld_vt & 7) == 0 && 8 * kVStep <= S) {
        int b, s;
        locate(m0 + (tid / BN) * 8, b, s);
        int64_t off = b * batch_stride + s;
        for (int g = tid / BN; g < BM / 8; g += kVStep) {
          const int r8 = g * 8;
          uint32_t p[4];
#pragma unroll
          for (int e = 0; e < 4; ++e)
            p[e] = static_cast<uint32_t>(sc[(r8 + 2 * e) * T::kLdc + cl]) |
                   (static_cast<uint32_t>(sc[(r8 + 2 * e + 1) * T::kLdc + cl]) << 16);
          *reinterpret_cast<u32x4*>(vrow + off) = u32x4{p[0], p[1], p[2], p[3]};
          s += 8 * kVStep;
          off += 8 * kVStep;
          const bool wrap = s >= S;
          s = wrap ? s - S : s;
          off = wrap ? off + batch_stride - S : off;
        }
      } else {
        for (int g = tid / BN; g < BM / 8; g += kVStep) {
          const int r8 = g * 8;
          const int row0 = m0 + r8;
          if (row0 >= M) break;
          int b0, s0;
          locate(row0, b0, s0);
          if (row0 + 7 < M && s0 + 7 < S && (s0 & 7) == 0 && (ep.ld_vt & 7) == 0) {
            uint32_t p[4];
#pragma unroll
            for (int e = 0; e < 4; ++e)
              p[e] = static_cast<uint32_t>(sc[(r8 + 2 * e) * T::kLdc + cl]) |
                     (static_cast<uint32_t>(sc[(r8 + 2 * e + 1) * T::kLdc + cl]) << 16);
            *reinterpret_cast<u32x4*>(vrow + b0 * batch_stride + s0) = u32x4{p[0], p[1], p[2], p[3]};
          } else {
            for (int e = 0; e < 8 && row0 + e < M; ++e) {
              int b, s;
              locate(row0 + e, b, s);
              vrow[b * batch_stride + s] = sc[(r8 + e) * T::kLdc + cl];
            }
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Skinny kernel for few rows (M <= 256): latency, not MFMA throughput, bounds
// these products, so the work is cut into many small independent pieces.
// v_mfma_f32_16x16x16_bf16 keeps the 16-deep K grouping of the 32x32x16 tiles
// above (the same accumulation as the library's kernels).  Lane layout:
//   A operand : row l%16, k = 4*(l/16) + j      (j = 0..3, 8 contiguous bytes)
//   B operand : col l%16, k = 4*(l/16) + j      (a W row, 8 contiguous bytes)
//   C/D       : col l%16, row = 4*(l/16) + j
// A and W stream through a two-stage LDS ring in K slices of KS = 256 (512
// bytes a row; KS = 128 when K is a multiple of 128 only, e.g. d_model 128)
// with direct global->LDS loads: one instruction moves 1 KiB of whole rows, so
// global reads are fully coalesced.  Inside a row the 16-byte chunk c sits in
// slot c ^ (row & 15), so the 16 rows one fragment read touches fall in
// distinct bank groups.
//   SPLIT == 1: 4 wavefronts, workgroup tile 16 x 64, wavefront w owns
//               columns 16w .. 16w+15 over the full K range in order.
//   SPLIT  > 1: SPLIT wavefronts, workgroup tile 16 x 16; K is cut into
//               CW-wide chunks and wavefront p accumulates chunks p, p+SPLIT,
//               ... (the library's split order); the partials meet in LDS and
//               are added in order before the bias.
constexpr int kSkinnyMaxRows = 256;  // products with at most this many rows use it

template <int EPI>
__device__ __forceinline__ void store_one(const GemmEpilogueArgs& ep, int N, int row, int col, float acc,
                                          float bias) {
  if constexpr (EPI == kEpiQkvHeadMajor) {
    const float y = acc + bias;
    const int D = ep.d_model, hd = ep.head_dim, S = ep.seq_len;
    const int which = col / D;
    const int rem = col - which * D;
    const int h = rem / hd;
    const int d = rem - h * hd;
    const int b = row / S;
    const int s = row - b * S;
    const int64_t bh = static_cast<int64_t>(b) * ep.num_heads + h;
    if (which < 2) {
      bf16_t* dst = which == 0 ? ep.q : ep.k;
      dst[(bh * S + s) * hd + d] = f32_to_bf16(y);
    } else {
      ep.v_t[(bh * hd + d) * ep.ld_vt + s] = f32_to_bf16(y);
    }
  } else {
    store_row_major<EPI>(ep, N, row, col, acc, bias);
  }
}

// R: LDS stages in the ring, all requested ahead (R - 1 in flight while one
// is multiplied)
template <int EPI, int SPLIT, int CW, int KS, int R = 2>
__global__ void __launch_bounds__(256)
gemm_skinny_kernel(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W, int M, int N, int K,
                   GemmEpilogueArgs ep) {
  constexpr int kWaves = SPLIT == 1 ? 4 : SPLIT;
  constexpr int kBN = SPLIT == 1 ? 64 : 16;
  constexpr int kRows = 16 + kBN;                       // LDS rows per stage (A then W)
  constexpr int kStage = kRows * KS;                    // elements per stage
  constexpr int kChunksRow = KS / 8;                    // 16-byte chunks per LDS row
  constexpr int kRowsPerLoad = kWave / kChunksRow;      // rows one load instruction fills
  constexpr int kLoads = kRows / kRowsPerLoad / kWaves;  // load instructions per wavefront
  constexpr int kStepsPerChunk = CW / 16;
  static_assert(KS == 128 || KS == 256, "stage width");
  static_assert(kRows % (kRowsPerLoad * kWaves) == 0, "load split");
  static_assert(SPLIT == 1 || (CW % 16 == 0 && KS % (CW * SPLIT) == 0), "chunk width");
  static_assert(R >= 2 && (R & (R - 1)) == 0 && (R - 1) * kLoads < 64, "ring depth");
  static_assert(R * kStage * 2 + SPLIT * 64 * 4 * 4 <= 160 * 1024, "LDS budget");
  __shared__ __attribute__((aligned(16))) bf16_t smem[R * kStage];
  __shared__ float red[SPLIT > 1 ? SPLIT : 1][64][4];

  const int tiles_m = (M + 15) / 16;
  // Tiles of one W column panel (the larger operand) are consecutive ids, and
  // each XCD (workgroups are dealt to the 8 XCDs round-robin) takes a
  // contiguous run of ids, so a panel is fetched into one XCD's L2 only.
  int id;
  {
    const int pid = blockIdx.x, num = gridDim.x;
    const int xcd = pid % kNumXcd, slot = pid / kNumXcd;
    id = xcd * (num / kNumXcd) + min(xcd, num % kNumXcd) + slot;
  }
  const int tm = id % tiles_m;
  const int tn = id / tiles_m;
  const int m0 = tm * 16;
  const int n0 = tn * kBN;
  const int lane = threadIdx.x % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);
  const int l16 = lane & 15;
  const int g = lane >> 4;

  // Load instruction j of wavefront w fills LDS rows R (kWaves j + w) .. +R-1
  // (R = rows per instruction); lane L writes slot L % C of row + L / C (C =
  // chunks per row), holding chunk (L % C) ^ (row & 15).
  const int ld_row = lane / kChunksRow;
  auto issue_stage = [&](int stage, int k0) {
    bf16_t* base = smem + stage * kStage;
#pragma unroll
    for (int j = 0; j < kLoads; ++j) {
      const int r0 = kRowsPerLoad * (kWaves * j + wave);
      const int r = r0 + ld_row;
      const int chunk = (lane % kChunksRow) ^ (r & 15);
      const bf16_t* src;
      if (r < 16) {
        src = A + static_cast<int64_t>(min(m0 + r, M - 1)) * K;  // rows past M: a valid row, never stored
      } else {
        src = W + static_cast<int64_t>(n0 + r - 16) * K;
      }
      __builtin_amdgcn_global_load_lds(src + k0 + chunk * 8, base + r0 * KS, 16, 0, 0);
    }
  };
  // fragment (8 bytes) of LDS row r at K-step s of the stage: chunk 2s + g/2
  auto frag = [&](int stage, int r, int s) {
    typedef short s16x4 __attribute__((ext_vector_type(4)));
    const int chunk = 2 * s + (g >> 1);
    const bf16_t* p = smem + stage * kStage + r * KS + ((chunk ^ (r & 15)) << 3) + 4 * (g & 1);
    return *reinterpret_cast<const s16x4*>(p);
  };

  const int wrow = 16 + (SPLIT == 1 ? wave * 16 : 0) + l16;  // this lane's W row in the stage
  // The epilogue's operands (bias, residual, row-mask bytes) do not depend on
  // the product: they are loaded before the K loop, so their latency overlaps
  // it instead of following the last MFMA.
  const int col = n0 + (SPLIT == 1 ? wave * 16 : 0) + l16;
  const float bias = bf16_to_f32(ep.bias[col]);
  constexpr bool kResidual = EPI == kEpiResidualKeep || EPI == kEpiResidualZero;
  // The values are held zero-extended in 32-bit registers and the mask
  // bytes untested until the epilogue: packing or testing them here would
  // make the wavefront wait for the loads before its K loop.
  uint32_t res[4] = {0u, 0u, 0u, 0u};
  uint32_t keep[4] = {1u, 1u, 1u, 1u};
  if constexpr (kResidual) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int r = min(m0 + 4 * g + j, M - 1);
      res[j] = ep.residual[static_cast<int64_t>(r) * N + col];
    }
    // without a mask the loads read the residual's first bytes (any valid
    // address) and the select below ignores them; a branch around the loads
    // would have the compiler test the bytes where the branch joins
    const bool has_mask = ep.row_mask != nullptr;
    const uint8_t* mask = has_mask ? ep.row_mask : reinterpret_cast<const uint8_t*>(ep.residual);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t byte = mask[has_mask ? min(m0 + 4 * g + j, M - 1) : 0];
      keep[j] = has_mask ? byte : 1u;
    }
  }
  f32x4 acc = {0.f, 0.f, 0.f, 0.f};
  const int nst = K / KS;
  if constexpr (R == 2) {
    issue_stage(0, 0);
    if (nst > 1) issue_stage(1, KS);
  } else {
#pragma unroll
    for (int st = 0; st < R; ++st)
      if (st < nst) issue_stage(st, st * KS);
  }
  for (int st = 0; st < nst; ++st) {
    const int buf = st & (R - 1);
    // the next R - 1 stages' loads may still be in flight (near the end,
    // fewer are left: wait for all)
    if (st + R - 1 < nst) {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm((R - 1) * kLoads, 0));
    } else {
      __builtin_amdgcn_s_waitcnt(waitcnt_imm(0, 0));
    }
    ring_barrier();
#pragma unroll
    for (int s = 0; s < KS / 16; ++s) {
      bool mine = true;
      if constexpr (SPLIT > 1) mine = ((s / kStepsPerChunk) % SPLIT) == wave;
      if (mine) acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(frag(buf, l16, s), frag(buf, wrow, s), acc, 0, 0, 0);
    }
    __builtin_amdgcn_s_waitcnt(waitcnt_imm(63, 0));
    ring_barrier();  // every wavefront is done reading this stage
    if (st + R < nst) issue_stage(buf, (st + R) * KS);
  }

  if constexpr (SPLIT > 1) {
#pragma unroll
    for (int j = 0; j < 4; ++j) red[wave][lane][j] = acc[j];
    __syncthreads();
    if (wave != 0) return;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      float sum = red[0][lane][j];
#pragma unroll
      for (int p = 1; p < SPLIT; ++p) sum += red[p][lane][j];
      acc[j] = sum;
    }
  }
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int r = m0 + 4 * g + j;
    if (r >= M) continue;
    if constexpr (kResidual) {
      const int64_t idx = static_cast<int64_t>(r) * N + col;
      const float y = round_bf16(acc[j] + bias);  // nn.Linear output boundary
      if (keep[j] != 0u) {
        ep.out[idx] = f32_to_bf16(__uint_as_float(res[j] << 16) + y);
      } else {
        ep.out[idx] = (EPI == kEpiResidualKeep) ? static_cast<bf16_t>(res[j]) : bf16_t(0);
      }
    } else {
      store_one<EPI>(ep, N, r, col, acc[j], bias);
    }
  }
}

template <int SPLIT, int CW, int KS, int R = 2>
hipError_t launch_skinny(const bf16_t* A, const bf16_t* W, int M, int N, int K, int epi,
                         const GemmEpilogueArgs& ep, hipStream_t st) {
  // K-split tiles (16 KiB stages) over more than two stages of K: four
  // stages, three in flight (c2's 128x512x2048 ffn_out 6.8 -> 6.15 us per
  // launch; eight stages gained less)
  if constexpr (SPLIT > 1 && R == 2) {
    if (K / KS > 2) return launch_skinny<SPLIT, CW, KS, 4>(A, W, M, N, K, epi, ep, st);
  }
  constexpr int kWaves = SPLIT == 1 ? 4 : SPLIT;
  constexpr int kBN = SPLIT == 1 ? 64 : 16;
  const dim3 grid(((M + 15) / 16) * (N / kBN)), block(kWaves * kWave);
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL((gemm_skinny_kernel<kEpiBias, SPLIT, CW, KS, R>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiBiasGelu: hipLaunchKernelGGL((gemm_skinny_kernel<kEpiBiasGelu, SPLIT, CW, KS, R>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualKeep: hipLaunchKernelGGL((gemm_skinny_kernel<kEpiResidualKeep, SPLIT, CW, KS, R>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualZero: hipLaunchKernelGGL((gemm_skinny_kernel<kEpiResidualZero, SPLIT, CW, KS, R>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiQkvHeadMajor: hipLaunchKernelGGL((gemm_skinny_kernel<kEpiQkvHeadMajor, SPLIT, CW, KS, R>), grid, block, 0, st, A, W, M, N, K, ep); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

struct TileShape {
  int bm, bn;
  int blocks_per_cu;  // resident workgroups per CU (LDS / register bound)
  float efficiency;   // relative MFMA efficiency of the tile shape
};

// 256x256 is not offered: with 4 wavefronts its 128x128 wave tiles need more
// than the 512 registers a lane has and spill.
constexpr TileShape kTiles[] = {
    {256, 128, 1, 0.85f},
    {128, 128, 2, 0.80f},
    {128, 64, 2, 0.62f},
    {64, 64, 4, 0.45f},
};

template <int BM, int BN>
hipError_t launch_tile(const bf16_t* A, const bf16_t* W, int M, int N, int K, int epi,
                       const GemmEpilogueArgs& ep, hipStream_t st) {
  const int tiles = ((M + BM - 1) / BM) * (N / BN);
  const dim3 grid(tiles), block(kThreads);
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, kEpiBias>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiBiasGelu: hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, kEpiBiasGelu>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualKeep: hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, kEpiResidualKeep>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualZero: hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, kEpiResidualZero>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiQkvHeadMajor:
      // The scattered head-major epilogue needs more registers than the two
      // largest tiles leave free (they would spill); it is limited to <= 128x128.
      if constexpr (BM * BN <= 128 * 128) {
        hipLaunchKernelGGL((gemm_bf16_kernel<BM, BN, kEpiQkvHeadMajor>), grid, block, 0, st, A, W, M, N, K, ep);
        break;
      } else {
        return hipErrorInvalidValue;
      }
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_narrow(const bf16_t* A, const bf16_t* W, int M, int N, int K, int epi,
                         const GemmEpilogueArgs& ep, hipStream_t st) {
  const int64_t blocks = static_cast<int64_t>((M + 31) / 32) * (N / 32);
  const dim3 grid(static_cast<uint32_t>((blocks + kThreads / kWave - 1) / (kThreads / kWave))), block(kThreads);
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL(gemm_narrow_kernel<kEpiBias>, grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiBiasGelu: hipLaunchKernelGGL(gemm_narrow_kernel<kEpiBiasGelu>, grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualKeep:
      hipLaunchKernelGGL(gemm_narrow_kernel<kEpiResidualKeep>, grid, block, 0, st, A, W, M, N, K, ep);
      break;
    case kEpiResidualZero:
      hipLaunchKernelGGL(gemm_narrow_kernel<kEpiResidualZero>, grid, block, 0, st, A, W, M, N, K, ep);
      break;
    case kEpiQkvHeadMajor:
      hipLaunchKernelGGL(gemm_narrow_kernel<kEpiQkvHeadMajor>, grid, block, 0, st, A, W, M, N, K, ep);
      break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// K-split launches use the 64x64 tile: four partial accumulator sets still fit
// the register budget there.
template <int SPLIT, int CW>
hipError_t launch_split(const bf16_t* A, const bf16_t* W, int M, int N, int K, int epi,
                        const GemmEpilogueArgs& ep, hipStream_t st) {
  const int tiles = ((M + 63) / 64) * (N / 64);
  const dim3 grid(tiles), block(kThreads);
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL((gemm_bf16_kernel<64, 64, kEpiBias, SPLIT, CW>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiBiasGelu: hipLaunchKernelGGL((gemm_bf16_kernel<64, 64, kEpiBiasGelu, SPLIT, CW>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualKeep: hipLaunchKernelGGL((gemm_bf16_kernel<64, 64, kEpiResidualKeep, SPLIT, CW>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualZero: hipLaunchKernelGGL((gemm_bf16_kernel<64, 64, kEpiResidualZero, SPLIT, CW>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiQkvHeadMajor: hipLaunchKernelGGL((gemm_bf16_kernel<64, 64, kEpiQkvHeadMajor, SPLIT, CW>), grid, block, 0, st, A, W, M, N, K, ep); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Enqueues the GELU table fill and its ready flag on the caller's stream
// before the device's first GELU product (no host synchronisation; products
// that run before the flag is set evaluate the erf).  Inside a stream capture
// the two launches are recorded into the graph, whose replays then refill
// the table, and the device stays unmarked so that a later uncaptured call
// fills it outside the graph.
std::mutex g_gelu_mutex;
bool g_gelu_enqueued[64] = {false};

hipError_t ensure_gelu_table(hipStream_t st) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  if (dev < 0 || dev >= 64) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> guard(g_gelu_mutex);
  if (g_gelu_enqueued[dev]) return hipSuccess;
  hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
  e = hipStreamIsCapturing(st, &capture);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(gelu_table_kernel, dim3(256), dim3(256), 0, st);
  hipLaunchKernelGGL(gelu_ready_kernel, dim3(1), dim3(1), 0, st);
  e = hipGetLastError();
  if (e == hipSuccess && capture == hipStreamCaptureStatusNone) g_gelu_enqueued[dev] = true;
  return e;
}

}  // namespace

hipError_t gemm_debug_gelu_table(int32_t ready, int32_t entry, int32_t value, hipStream_t st) {
  hipError_t e = ensure_gelu_table(st);
  if (e != hipSuccess) return e;
  if (entry >= 0) hipLaunchKernelGGL(gelu_entry_set_kernel, dim3(1), dim3(1), 0, st, static_cast<uint32_t>(entry), value);
  if (ready >= 0) hipLaunchKernelGGL(gelu_flag_set_kernel, dim3(1), dim3(1), 0, st, static_cast<uint32_t>(ready));
  return hipGetLastError();
}

namespace {

template <int BM, int BN, int BK, int NS, int OCC = 1>
hipError_t launch_big(const bf16_t* A, const bf16_t* W, int M, int N, int K, int epi,
                      const GemmEpilogueArgs& ep, hipStream_t st) {
  if (epi == kEpiBiasGelu) {
    const hipError_t e = ensure_gelu_table(st);
    if (e != hipSuccess) return e;
  }
  const int tiles = ((M + BM - 1) / BM) * (N / BN);
  const dim3 grid(tiles), block(kThreads);
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL((gemm_big_kernel<BM, BN, BK, NS, kEpiBias, OCC>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiBiasGelu: hipLaunchKernelGGL((gemm_big_kernel<BM, BN, BK, NS, kEpiBiasGelu, OCC>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualKeep: hipLaunchKernelGGL((gemm_big_kernel<BM, BN, BK, NS, kEpiResidualKeep, OCC>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiResidualZero: hipLaunchKernelGGL((gemm_big_kernel<BM, BN, BK, NS, kEpiResidualZero, OCC>), grid, block, 0, st, A, W, M, N, K, ep); break;
    case kEpiQkvHeadMajor: hipLaunchKernelGGL((gemm_big_kernel<BM, BN, BK, NS, kEpiQkvHeadMajor, OCC>), grid, block, 0, st, A, W, M, N, K, ep); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// ---------------------------------------------------------------------------
// Stream-K tail.  For the shapes in streamk_tail.h the library accumulates its
// last 256 x 256 output tiles in two partial sums, K < s and K >= s (s per
// tile, measured), and adds them before the bias.  This kernel computes those
// rows the same way: 128 x 128 workgroup tiles (each inside one library tile),
// sequential 16-deep MFMA steps inside each partial, then
//   y = bf16((P1 + P2) + bias)          (s > 0)
//   y = bf16(P + bias)                  (s == 0: one pass, as elsewhere)
// through the usual epilogue.  Only the tail rows run here (0.6% of c5's rows),
// so the kernel stages operands through registers and LDS plainly.
constexpr int kTailMaxTiles = 1024;  // 2 KiB of kernel arguments
struct TailSplitArgs {
  int row_begin;   // first row of the tail, a multiple of 256
  int slice_n;     // N of the library product the table describes
  int tile_cols;   // 256-wide tiles per slice
  uint16_t split[kTailMaxTiles];
};

template <int EPI>
__global__ void __launch_bounds__(kThreads)
gemm_tail_split_kernel(const bf16_t* __restrict__ A, const bf16_t* __restrict__ W, int M, int N, int K,
                       TailSplitArgs ts, GemmEpilogueArgs ep) {
  constexpr int BM = 128, BN = 128, RM = 2, RN = 2;
  constexpr int A_LOADS = BM * (kBK / 8) / kThreads;
  constexpr int B_LOADS = BN * (kBK / 8) / kThreads;
  __shared__ __attribute__((aligned(16))) bf16_t sA[2][BM * kLdk];
  __shared__ __attribute__((aligned(16))) bf16_t sB[2][BN * kLdk];

  const int tiles_n = N / BN;
  const int tm = blockIdx.x / tiles_n;
  const int tn = blockIdx.x - tm * tiles_n;
  const int m0 = ts.row_begin + tm * BM;
  const int n0 = tn * BN;
  const int lib_row = (m0 - ts.row_begin) / 256;
  const int lib_col = (n0 % ts.slice_n) / 256;
  const int split = ts.split[lib_row * ts.tile_cols + lib_col];

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = tid / kWave;
  const int wm = wave >> 1;
  const int wn = wave & 1;
  const int l32 = lane & 31;
  const int lhi = lane >> 5;

  u32x4 ra[A_LOADS];
  u32x4 rb[B_LOADS];
  auto load_global = [&](int k0) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int c = tid + i * kThreads;
      const int grow = min(m0 + (c >> 3), M - 1);  // rows past M are never stored
      ra[i] = *reinterpret_cast<const u32x4*>(A + static_cast<int64_t>(grow) * K + k0 + (c & 7) * 8);
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int c = tid + i * kThreads;
      rb[i] = *reinterpret_cast<const u32x4*>(W + static_cast<int64_t>(n0 + (c >> 3)) * K + k0 + (c & 7) * 8);
    }
  };
  auto store_lds = [&](int buf) {
#pragma unroll
    for (int i = 0; i < A_LOADS; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(&sA[buf][(c >> 3) * kLdk + (c & 7) * 8]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < B_LOADS; ++i) {
      const int c = tid + i * kThreads;
      *reinterpret_cast<u32x4*>(&sB[buf][(c >> 3) * kLdk + (c & 7) * 8]) = rb[i];
    }
  };

  f32x16 p1[RM][RN], p2[RM][RN];
#pragma unroll
  for (int i = 0; i < RM; ++i)
#pragma unroll
    for (int j = 0; j < RN; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        p1[i][j][r] = 0.f;
        p2[i][j][r] = 0.f;
      }

  const int KT = K / kBK;
  load_global(0);
  store_lds(0);
  __syncthreads();
  const int a_base = (wm * (BM / 2) + l32) * kLdk + lhi * 8;
  const int b_base = (wn * (BN / 2) + l32) * kLdk + lhi * 8;
  for (int kt = 0; kt < KT; ++kt) {
    const int cur = kt & 1;
    if (kt + 1 < KT) load_global((kt + 1) * kBK);
    const bool second = kt * kBK >= split;  // uniform: which partial this K block feeds
#pragma unroll
    for (int ks = 0; ks < kBK / 16; ++ks) {
      bf16x8 af[RM], bfr[RN];
#pragma unroll
      for (int i = 0; i < RM; ++i)
        af[i] = *reinterpret_cast<const bf16x8*>(&sA[cur][a_base + i * 32 * kLdk + ks * 16]);
#pragma unroll
      for (int j = 0; j < RN; ++j)
        bfr[j] = *reinterpret_cast<const bf16x8*>(&sB[cur][b_base + j * 32 * kLdk + ks * 16]);
      if (second) {
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
          for (int j = 0; j < RN; ++j)
            p2[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], p2[i][j], 0, 0, 0);
      } else {
#pragma unroll
        for (int i = 0; i < RM; ++i)
#pragma unroll
          for (int j = 0; j < RN; ++j)
            p1[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bfr[j], p1[i][j], 0, 0, 0);
      }
    }
    if (kt + 1 < KT) store_lds(cur ^ 1);
    __syncthreads();
  }

  const int row_base = m0 + wm * (BM / 2);
  const int col_base = n0 + wn * (BN / 2);
#pragma unroll
  for (int j = 0; j < RN; ++j) {
    const int col = col_base + j * 32 + l32;
    const float bias = bf16_to_f32(ep.bias[col]);
#pragma unroll
    for (int i = 0; i < RM; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int row = row_base + i * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
        if (row >= M) continue;
        // (P1 + P2) + bias, matched bitwise against the library on random
        // inputs; the other orders, P1 + (P2 + bias) and (P1 + bias) + P2,
        // were measured to differ.  With no split every K block went to p2.
        const float sum = split == 0 ? p2[i][j][r] : p1[i][j][r] + p2[i][j][r];
        store_one<EPI>(ep, N, row, col, sum, bias);
      }
    }
  }
}

// Reduction orders measured on the running device and registered by the host
// (enc_linear_order_register): per device and library product shape
// (M, N, K), either "sequential" (no tile of the library's product has its K
// range split) or a tail table in the StreamKTail layout.  They take
// precedence over the built-in tables below, which were measured on a 256-CU
// MI355X and apply only on a device with that many CUs.
struct RegisteredOrder {
  int device;
  int64_t m;
  int n, k;
  int first_tile_row, tile_rows, tile_cols;
  std::vector<uint16_t> split;  // empty: sequential
};
std::mutex g_order_mutex;
std::vector<RegisteredOrder> g_orders;

// What gemm_bf16 uses for one product: no split, or a copy of a tail table.
struct TailLookup {
  bool split = false;
  int64_t m = 0;
  int n = 0, k = 0;
  int first_tile_row = 0, tile_rows = 0, tile_cols = 0;
  uint16_t table[kTailMaxTiles] = {};
};

// The packed QKV projection (N = 3 x slice_n, head-major epilogue) matches a
// slice_n entry: the reference runs the q, k and v projections as three
// [M, K] x [slice_n, K]^T products.
bool order_matches(int64_t tm, int64_t tn, int64_t tk, int64_t M, int64_t N, int64_t K, int epi) {
  return tm == M && tk == K && (N == tn || (epi == kEpiQkvHeadMajor && N == 3 * tn));
}

void lookup_order(int64_t M, int64_t N, int64_t K, int epi, int num_cus, TailLookup* out) {
  out->split = false;
  int dev = -1;
  if (hipGetDevice(&dev) == hipSuccess) {
    std::lock_guard<std::mutex> guard(g_order_mutex);
    for (const RegisteredOrder& r : g_orders) {
      if (r.device != dev || !order_matches(r.m, r.n, r.k, M, N, K, epi)) continue;
      if (r.split.empty()) return;
      out->split = true;
      out->m = r.m;
      out->n = r.n;
      out->k = r.k;
      out->first_tile_row = r.first_tile_row;
      out->tile_rows = r.tile_rows;
      out->tile_cols = r.tile_cols;
      std::copy(r.split.begin(), r.split.end(), out->table);
      return;
    }
  }
  if (num_cus != kStreamKTablesCUs) return;
  for (const StreamKTail& t : kStreamKTails) {
    if (!order_matches(t.m, t.n, t.k, M, N, K, epi)) continue;
    out->split = true;
    out->m = t.m;
    out->n = t.n;
    out->k = t.k;
    out->first_tile_row = t.first_tile_row;
    out->tile_rows = t.tile_rows;
    out->tile_cols = t.tile_cols;
    std::copy(t.split, t.split + t.tile_rows * t.tile_cols, out->table);
    return;
  }
}

hipError_t launch_tail_split(const bf16_t* A, const bf16_t* W, int M, int N, int K, int epi,
                             const TailLookup& t, const GemmEpilogueArgs& ep, hipStream_t st) {
  TailSplitArgs ts;
  ts.row_begin = t.first_tile_row * 256;
  ts.slice_n = t.n;
  ts.tile_cols = t.tile_cols;
  const int entries = t.tile_rows * t.tile_cols;
  if (entries > kTailMaxTiles || t.tile_cols * 256 != t.n || N % 128 != 0) return hipErrorInvalidValue;
  for (int i = 0; i < kTailMaxTiles; ++i) ts.split[i] = i < entries ? t.table[i] : 0;
  const int rows = M - ts.row_begin;
  const dim3 grid(static_cast<uint32_t>((rows + 127) / 128 * (N / 128))), block(kThreads);
  switch (epi) {
    case kEpiBias: hipLaunchKernelGGL(gemm_tail_split_kernel<kEpiBias>, grid, block, 0, st, A, W, M, N, K, ts, ep); break;
    case kEpiBiasGelu: hipLaunchKernelGGL(gemm_tail_split_kernel<kEpiBiasGelu>, grid, block, 0, st, A, W, M, N, K, ts, ep); break;
    case kEpiResidualKeep: hipLaunchKernelGGL(gemm_tail_split_kernel<kEpiResidualKeep>, grid, block, 0, st, A, W, M, N, K, ts, ep); break;
    case kEpiResidualZero: hipLaunchKernelGGL(gemm_tail_split_kernel<kEpiResidualZero>, grid, block, 0, st, A, W, M, N, K, ts, ep); break;
    case kEpiQkvHeadMajor: hipLaunchKernelGGL(gemm_tail_split_kernel<kEpiQkvHeadMajor>, grid, block, 0, st, A, W, M, N, K, ts, ep); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

// Tile of the large-tile kernel for this shape, or 0 when the small-tile
// kernel should run: the operands must be 16-byte aligned (16-byte loads per
// lane), the residual / outputs too (16-byte epilogue stores), and the tile
// count should fill the device's CUs.
int pick_big_tile(int64_t M, int64_t N, const bf16_t* A, const bf16_t* W, const GemmEpilogueArgs& ep,
                  bool ep_overlaps, int num_cus) {
  auto al = [](const void* p) { return reinterpret_cast<uintptr_t>(p) % 16 == 0; };
  if (!al(A) || !al(W) || !al(ep.out) || !al(ep.residual) || !al(ep.q) || !al(ep.k) || !al(ep.v_t) ||
      !al(ep.w_packed) || reinterpret_cast<uintptr_t>(ep.bias) % 8 != 0)  // 8-byte bias loads
    return 0;
  if (M < 1024) return 0;
  const int64_t t256x128 = ((M + 255) / 256) * (N / 128);
  // With two resident 256x128 tiles per CU one tile's epilogue overlaps the
  // other's MFMA loop (when there are tiles for two per CU: a narrow N leaves
  // most CUs idle).  It pays where the epilogue is long against the K loop:
  // the GELU (32768x4096x1024: 314 vs 366 us on 256x256 tiles).  The
  // residual epilogues run as fast or faster on the 256x256 tiles
  // (32768x1024x1024 plain weight: 73.5 vs 83.2 us; 409600x1024x1024 packed:
  // 932 vs 1007 us).
  if (ep_overlaps && N % 128 == 0 && t256x128 >= 2 * num_cus) return 256129;
  // Whole rounds of tiles over the CUs times the tile's work, over its
  // measured per-tile efficiency (256x128 tiles run ~10% below 256x256).
  auto cost = [&](int bm, int bn, double eff) {
    const int64_t tiles = ((M + bm - 1) / bm) * (N / bn);
    const int64_t rounds = (tiles + num_cus - 1) / num_cus;
    return static_cast<double>(rounds) * bm * bn / eff;
  };
  if (N % 256 == 0 && cost(256, 256, 1.0) <= cost(256, 128, 0.9)) return 256256;
  if (N % 128 == 0 && t256x128 >= num_cus) return 256128;
  if (N % 128 == 0) return 128128;
  return 0;
}

}  // namespace

namespace {

// One 16-byte chunk (8 elements of one row) per thread: reads are row-major
// W, writes land in the packed order.
__global__ void __launch_bounds__(256)
gemm_prepack_kernel(const bf16_t* __restrict__ W, bf16_t* __restrict__ P, int N, int K, int pn) {
  const int64_t chunk = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
  const int chunks_per_row = K / 8;
  if (chunk >= static_cast<int64_t>(N) * chunks_per_row) return;
  const int n = static_cast<int>(chunk / chunks_per_row);
  const int k = static_cast<int>(chunk - static_cast<int64_t>(n) * chunks_per_row) * 8;
  const int64_t dst = ((static_cast<int64_t>(n / pn) * (K / 32) + k / 32) * pn + n % pn) * 32 + k % 32;
  *reinterpret_cast<u32x4*>(P + dst) = *reinterpret_cast<const u32x4*>(W + static_cast<int64_t>(n) * K + k);
}

}  // namespace

int gemm_prepack_rows(int64_t N, int64_t K) {
  if (N <= 0 || K <= 0 || K % 32 != 0) return 0;
  if (N % 256 == 0) return 256;
  if (N % 128 == 0) return 128;
  return 0;
}

hipError_t gemm_prepack_weight(const bf16_t* W, bf16_t* packed, int64_t N, int64_t K, hipStream_t stream) {
  const int pn = gemm_prepack_rows(N, K);
  if (pn == 0 || N * K > (int64_t(1) << 31)) return hipErrorInvalidValue;
  const int64_t chunks = N * (K / 8);
  hipLaunchKernelGGL(gemm_prepack_kernel, dim3(static_cast<uint32_t>((chunks + 255) / 256)), dim3(256), 0, stream, W,
                     packed, static_cast<int>(N), static_cast<int>(K), pn);
  return hipGetLastError();
}

void gemm_split_plan(int64_t M, int64_t N, int64_t K, int* split, int* chunk) {
  // The reduction order torch.nn.functional.linear (hipBLASLt on ROCm 7) uses
  // for bf16 [M, K] x [N, K]^T, measured per shape with inputs whose rounding
  // reveals which K indices share a partial sum.  Shapes not listed here
  // accumulate K sequentially, which is what the unsplit kernel does.
  struct Rule {
    int64_t max_m, n, k;
    int split, chunk;
  };
  static constexpr Rule kRules[] = {
      {16, 512, 512, 4, 32},    {16, 512, 2048, 4, 32},   {16, 1536, 512, 4, 32},
      {16, 2048, 512, 4, 32},   {16, 1024, 1024, 4, 32},  {16, 1024, 4096, 2, 128},
      {16, 4096, 1024, 4, 32},  {16, 3072, 1024, 4, 32},  {64, 512, 2048, 4, 32},
      {64, 1024, 4096, 2, 128}, {128, 512, 2048, 4, 32},  {128, 1024, 4096, 4, 64},
      {256, 512, 2048, 4, 32},
  };
  *split = 1;
  *chunk = kBK;
  for (const Rule& r : kRules) {
    if (M <= r.max_m && N == r.n && K == r.k) {
      *split = r.split;
      *chunk = r.chunk;
      return;
    }
  }
}

void gemm_pick_tile(int64_t M, int64_t N, int epilogue, int num_cus, int* bm, int* bn) {
  double best = 1e300;
  *bm = 64;
  *bn = 64;
  for (const TileShape& t : kTiles) {
    if (N % t.bn != 0) continue;
    if (epilogue == kEpiQkvHeadMajor && t.bm * t.bn > 128 * 128) continue;
    const int64_t tiles = ((M + t.bm - 1) / t.bm) * (N / t.bn);
    const int64_t slots = static_cast<int64_t>(num_cus) * t.blocks_per_cu;
    const int64_t rounds = (tiles + slots - 1) / slots;
    // A round runs blocks_per_cu tiles side by side on every CU, sharing its
    // MFMA pipes: time ~ rounds * blocks_per_cu * (tile work) / efficiency.
    const double cost = static_cast<double>(rounds) * t.blocks_per_cu * t.bm * t.bn / t.efficiency;
    if (cost < best * 0.999) {
      best = cost;
      *bm = t.bm;
      *bn = t.bn;
    }
  }
}

bool gemm_supported(int64_t M, int64_t N, int64_t K) {
  return M >= 0 && N > 0 && K > 0 && N % 32 == 0 && K % 32 == 0 && M < (int64_t(1) << 31) &&
         N < (int64_t(1) << 20) && K < (int64_t(1) << 20);
}

namespace {

// The product without the stream-K tail rule: every tile in one pass (or the
// small-M split plan).
hipError_t gemm_bf16_plain(const bf16_t* A, const bf16_t* W, int64_t M, int64_t N, int64_t K, int epi,
                           const GemmEpilogueArgs& ep, int num_cus, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  // N or K not a multiple of 64: one 32x32 block per wavefront, sequential K
  // (none of these shapes has a split rule)
  if (N % 64 != 0 || K % 64 != 0) return launch_narrow(A, W, m, n, k, epi, ep, stream);
  int split, chunk;
  gemm_split_plan(M, N, K, &split, &chunk);
  const bool aligned16 = reinterpret_cast<uintptr_t>(A) % 16 == 0 && reinterpret_cast<uintptr_t>(W) % 16 == 0;
  // whole LDS stages, each holding whole rounds of the split's chunks
  const bool whole = K % 256 == 0 && 256 % (chunk * split) == 0;
  // With K <= 256 (d_model 128 or 256) a product stays latency-bound well past
  // 256 rows, and the 16-row tiles put the most workgroups in flight: up to
  // 2048 rows, and up to 8192 rows for N <= 128 (measured on MI355X against
  // the large tiles and the 64x64 tiles).
  const bool skinny_rows = M <= kSkinnyMaxRows || (K <= 256 && (M <= 2048 || (N <= 128 && M <= 8192)));
  if (skinny_rows && aligned16 && whole) {
    if (split == 1) return launch_skinny<1, 16, 256>(A, W, m, n, k, epi, ep, stream);
    if (split == 4 && chunk == 32) return launch_skinny<4, 32, 256>(A, W, m, n, k, epi, ep, stream);
    if (split == 4 && chunk == 64) return launch_skinny<4, 64, 256>(A, W, m, n, k, epi, ep, stream);
    if (split == 2 && chunk == 128) return launch_skinny<2, 128, 256>(A, W, m, n, k, epi, ep, stream);
  }
  // K a multiple of 128 only (d_model 128): 128-wide stages, sequential K
  if (skinny_rows && aligned16 && split == 1 && K % 128 == 0)
    return launch_skinny<1, 16, 128>(A, W, m, n, k, epi, ep, stream);
  if (split == 4 && chunk == 32) return launch_split<4, 32>(A, W, m, n, k, epi, ep, stream);
  if (split == 4 && chunk == 64) return launch_split<4, 64>(A, W, m, n, k, epi, ep, stream);
  if (split == 2 && chunk == 128) return launch_split<2, 128>(A, W, m, n, k, epi, ep, stream);
  const bool ep_overlaps = epi == kEpiBiasGelu;
  // The large-tile head-major epilogue stores 8 channels of one head at a
  // time (Q, K) and channel pairs (V^T): head_dim must be a multiple of 8.
  const bool big_ok = epi != kEpiQkvHeadMajor || ep.head_dim % 8 == 0;
  switch (big_ok ? pick_big_tile(M, N, A, W, ep, ep_overlaps, num_cus) : 0) {
    case 256129: return launch_big<256, 128, 32, 3, 2>(A, W, m, n, k, epi, ep, stream);
    // 256x256 tiles: from the plain nn.Linear weight, 64-deep K blocks in two
    // stages (32768x3072x1024: 190 vs 201 us); from the tile-packed copy,
    // whose 32-deep slices make each load one 1 KiB run, 32-deep blocks in
    // four stages (197 vs 225 us).  A/B in one process, bitwise the same.
    case 256256:
      if (ep.w_packed != nullptr) return launch_big<256, 256, 32, 4>(A, W, m, n, k, epi, ep, stream);
      return launch_big<256, 256, 64, 2>(A, W, m, n, k, epi, ep, stream);
    case 256128: return launch_big<256, 128, 64, 3>(A, W, m, n, k, epi, ep, stream);
    case 128128: return launch_big<128, 128, 64, 3>(A, W, m, n, k, epi, ep, stream);
    default: break;
  }
  int bm, bn;
  gemm_pick_tile(M, N, epi, num_cus, &bm, &bn);
  if (bm == 256 && bn == 128) return launch_tile<256, 128>(A, W, m, n, k, epi, ep, stream);
  if (bm == 128 && bn == 128) return launch_tile<128, 128>(A, W, m, n, k, epi, ep, stream);
  if (bm == 128 && bn == 64) return launch_tile<128, 64>(A, W, m, n, k, epi, ep, stream);
  return launch_tile<64, 64>(A, W, m, n, k, epi, ep, stream);
}

}  // namespace

hipError_t gemm_bf16(const bf16_t* A, const bf16_t* W, int64_t M, int64_t N, int64_t K, int epi,
                     const GemmEpilogueArgs& ep, int num_cus, hipStream_t stream) {
  // a packed copy must be the one gemm_prepack_weight writes for this shape
  if (ep.w_packed != nullptr && ep.w_packed_rows != gemm_prepack_rows(N, K)) return hipErrorInvalidValue;
  TailLookup tail;
  lookup_order(M, N, K, epi, num_cus, &tail);
  if (!tail.split) return gemm_bf16_plain(A, W, M, N, K, epi, ep, num_cus, stream);
  // rows before the library's stream-K tail as usual, the tail's rows split
  const int64_t row_begin = static_cast<int64_t>(tail.first_tile_row) * 256;
  hipError_t e = gemm_bf16_plain(A, W, row_begin, N, K, epi, ep, num_cus, stream);
  if (e != hipSuccess) return e;
  return launch_tail_split(A, W, static_cast<int>(M), static_cast<int>(N), static_cast<int>(K), epi, tail, ep, stream);
}

bool gemm_has_split_tail(int64_t M, int64_t N, int64_t K, int num_cus) {
  TailLookup tail;
  lookup_order(M, N, K, kEpiBias, num_cus, &tail);
  return tail.split;
}

int gemm_order_register(int device, int64_t M, int64_t N, int64_t K, int first_tile_row, int tile_rows,
                        int tile_cols, const uint16_t* split) {
  if (M <= 0 || N <= 0 || K <= 0 || tile_rows < 0 || first_tile_row < 0) return 1;
  if (tile_rows > 0) {
    if (split == nullptr || N % 256 != 0 || tile_cols != N / 256 || tile_rows * tile_cols > kTailMaxTiles ||
        (static_cast<int64_t>(first_tile_row) + tile_rows) * 256 < M ||
        static_cast<int64_t>(first_tile_row) * 256 >= M)
      return 1;
    for (int i = 0; i < tile_rows * tile_cols; ++i)
      if (split[i] >= K || split[i] % 32 != 0) return 1;
  }
  RegisteredOrder r;
  r.device = device;
  r.m = M;
  r.n = static_cast<int>(N);
  r.k = static_cast<int>(K);
  r.first_tile_row = first_tile_row;
  r.tile_rows = tile_rows;
  r.tile_cols = tile_rows > 0 ? tile_cols : 0;
  if (tile_rows > 0) r.split.assign(split, split + tile_rows * tile_cols);
  std::lock_guard<std::mutex> guard(g_order_mutex);
  for (RegisteredOrder& o : g_orders) {
    if (o.device == device && o.m == M && o.n == N && o.k == K) {
      o = std::move(r);
      return 0;
    }
  }
  g_orders.push_back(std::move(r));
  return 0;
}

void gemm_order_clear() {
  std::lock_guard<std::mutex> guard(g_order_mutex);
  g_orders.clear();
}

}  // namespace enc
