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
#include "common.h"
#include "kernels.h"

namespace enc {

namespace {

constexpr int kBK = 64;
constexpr int kLdk = kBK + 8;  // padded LDS row, elements
constexpr int kThreads = 256;
constexpr int kNumXcd = 8;
constexpr int kGroupM = 8;

__device__ __forceinline__ void map_tile(int tiles_m, int tiles_n, int* tm, int* tn) {
  const int num = tiles_m * tiles_n;
  int pid = blockIdx.x;
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
  map_tile(tiles_m, tiles_n, &tm, &tn);
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
    const int col = col_base + j * 32 + l32;
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
      for (int i = 0; i < RM; ++i) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const int row0 = row_base + i * 32 + 8 * g + 4 * lhi;  // 4 consecutive rows
          float y[4];
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) y[jj] = acc[0][i][j][4 * g + jj] + bias;
          if (which < 2) {
            bf16_t* dst = which == 0 ? ep.q : ep.k;
#pragma unroll
            for (int jj = 0; jj < 4; ++jj) {
              const int row = row0 + jj;
              if (row < M) {
                const int b = row / S;
                const int s = row - b * S;
                dst[((static_cast<int64_t>(b) * ep.num_heads + h) * S + s) * hd + d] = f32_to_bf16(y[jj]);
              }
            }
          } else {
            const int b0 = row0 / S;
            const int s0 = row0 - b0 * S;
            if (row0 + 3 < M && s0 + 3 < S && (ep.ld_vt & 3) == 0 && (s0 & 3) == 0) {
              bf16_t* dst = ep.v_t + ((static_cast<int64_t>(b0) * ep.num_heads + h) * hd + d) * ep.ld_vt + s0;
              u32x2 w = {pack_bf16x2(y[0], y[1]), pack_bf16x2(y[2], y[3])};
              *reinterpret_cast<u32x2*>(dst) = w;
            } else {
#pragma unroll
              for (int jj = 0; jj < 4; ++jj) {
                const int row = row0 + jj;
                if (row < M) {
                  const int b = row / S;
                  const int s = row - b * S;
                  ep.v_t[((static_cast<int64_t>(b) * ep.num_heads + h) * hd + d) * ep.ld_vt + s] = f32_to_bf16(y[jj]);
                }
              }
            }
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < RM; ++i) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int row = row_base + i * 32 + 8 * (r >> 2) + 4 * lhi + (r & 3);
          if (row < M) store_row_major<EPI>(ep, N, row, col, acc[0][i][j][r], bias);
        }
      }
    }
  }
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

}  // namespace

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
  return M >= 0 && N > 0 && K > 0 && N % 64 == 0 && K % 64 == 0 && M < (int64_t(1) << 31) &&
         N < (int64_t(1) << 20) && K < (int64_t(1) << 20);
}

hipError_t gemm_bf16(const bf16_t* A, const bf16_t* W, int64_t M, int64_t N, int64_t K, int epi,
                     const GemmEpilogueArgs& ep, int num_cus, hipStream_t stream) {
  if (M == 0) return hipSuccess;
  const int m = static_cast<int>(M), n = static_cast<int>(N), k = static_cast<int>(K);
  int split, chunk;
  gemm_split_plan(M, N, K, &split, &chunk);
  if (split == 4 && chunk == 32) return launch_split<4, 32>(A, W, m, n, k, epi, ep, stream);
  if (split == 4 && chunk == 64) return launch_split<4, 64>(A, W, m, n, k, epi, ep, stream);
  if (split == 2 && chunk == 128) return launch_split<2, 128>(A, W, m, n, k, epi, ep, stream);
  int bm, bn;
  gemm_pick_tile(M, N, epi, num_cus, &bm, &bn);
  if (bm == 256 && bn == 128) return launch_tile<256, 128>(A, W, m, n, k, epi, ep, stream);
  if (bm == 128 && bn == 128) return launch_tile<128, 128>(A, W, m, n, k, epi, ep, stream);
  if (bm == 128 && bn == 64) return launch_tile<128, 64>(A, W, m, n, k, epi, ep, stream);
  return launch_tile<64, 64>(A, W, m, n, k, epi, ep, stream);
}

}  // namespace enc
