// LayerNorm for bf16 activations with PyTorch-on-ROCm bit-exact statistics.
//
// One 64-lane wavefront owns one row (HBM-bound: the row is read once and
// written once).  The statistics reproduce, operation for operation, the
// vectorised Welford LayerNorm that torch's native nn.LayerNorm runs on ROCm
// for bf16 rows whose width is a multiple of 4, so the bf16 output is bitwise
// identical to the reference's (models.py:721, 723, 907):
//   * the row is viewed as width/4 vectors of 4 elements; "virtual thread" t of
//     a 256-thread block (4 warps x 64 lanes) folds vectors t, t+256, ... with
//     Welford online updates  mean += delta * rcp(n);  m2 += delta * (x - mean)
//     (FMA on the mean update only).  rcp is the hardware v_rcp_f32, which
//     is not the correctly rounded 1/n for every n (1/3 comes out one ulp
//     low), so it is issued through inline asm: with the counts known at
//     compile time the builtin would be folded to the correctly rounded value;
//   * each virtual warp is merged by a shuffle-down tree (offsets 32..1) of the
//     Welford combine (count-weighted mean, m2 += delta^2 * nA * nB / n), then
//     warps 0+2, 1+3 and 0+1;
//   * var = m2 / width, rstd = rsqrt(var + eps), y = fma(gamma, rstd*(x-mean), beta).
// Here lane l carries virtual threads l, l+64, l+128, l+192 (one per virtual
// warp) and runs the four warp trees side by side.  The operation order was
// pinned against torch's native_layer_norm on an MI355X: mean and rstd of
// 4096 encoder activation rows (width 1024) and of 24576 rows built to expose
// the merge order all agree bit for bit.
#include "common.h"
#include "kernels.h"
#include "welford.h"

namespace enc {

namespace {

constexpr int kRowsPerBlock = 4;  // one row per wavefront, 4 wavefronts

// WIDTH = row width; the row is WIDTH/4 vectors, lane l holds vectors
// l + 64 s (s < SLOTS).  Narrow rows (WIDTH < 256) leave lanes and whole
// virtual warps without a vector: their Welford states stay at count 0 and
// still take part in the merges, as the idle threads of the reference's
// 256-thread block do.
template <int WIDTH>
__global__ void __launch_bounds__(kRowsPerBlock * kWave)
layernorm_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ gamma,
                 const bf16_t* __restrict__ beta, bf16_t* __restrict__ y, int64_t rows, float eps,
                 const uint8_t* __restrict__ row_mask) {
  constexpr int kVecs = WIDTH / 4;
  constexpr int kSlots = kVecs < kWave ? 1 : kVecs / kWave;  // vectors per lane
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const bf16_t* xr = x + row * WIDTH;
  bf16_t* yr = y + row * WIDTH;
  const bool has = kVecs >= kWave || lane < kVecs;  // this lane holds vectors

  // slot s <-> vector index v = lane + 64*s, i.e. virtual thread t = v % 256
  // (virtual warp w = (v / 64) % 4) and its (v / 256)-th vector.
  float v[kSlots][4];
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    u32x2 w = {0u, 0u};
    if (has) w = *reinterpret_cast<const u32x2*>(xr + (lane + kWave * s) * 4);
    v[s][0] = lo_bf16(w[0]);
    v[s][1] = hi_bf16(w[0]);
    v[s][2] = lo_bf16(w[1]);
    v[s][3] = hi_bf16(w[1]);
  }
  // gamma and beta: at widths >= 1024 requested with the row, so their
  // latency overlaps the statistics (8192 rows of 1024: 9.3 -> 8.35 us); the
  // narrower rows' short statistics measured no gain from it
  constexpr bool kEarlyAffine = WIDTH >= 1024;
  u32x2 gw[kSlots], bw[kSlots];
  auto load_affine = [&]() {
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      gw[s] = u32x2{0u, 0u};
      bw[s] = u32x2{0u, 0u};
      if (has) {
        gw[s] = *reinterpret_cast<const u32x2*>(gamma + (lane + kWave * s) * 4);
        bw[s] = *reinterpret_cast<const u32x2*>(beta + (lane + kWave * s) * 4);
      }
    }
  };
  if constexpr (kEarlyAffine) load_affine();

  if (row_mask != nullptr && row_mask[row] == 0) {
    if (has) {
#pragma unroll
      for (int s = 0; s < kSlots; ++s)
        *reinterpret_cast<u32x2*>(yr + (lane + kWave * s) * 4) = u32x2{0u, 0u};
    }
    return;
  }

  // Welford per virtual warp (one state per virtual thread = this lane in warp w)
  Welford st[4];
#pragma unroll
  for (int w = 0; w < 4; ++w) st[w] = {0.f, 0.f, 0.f};
  if (has) {
#pragma unroll
    for (int s = 0; s < kSlots; ++s) {
      const int w = s % 4;  // vector v = lane + 64 s belongs to virtual warp s % 4
#pragma unroll
      for (int e = 0; e < 4; ++e) st[w] = welford_add(st[w], v[s][e]);
    }
  }
  float mean_all, m2_all;
  if constexpr (WIDTH >= 1024) {
    // Every virtual thread holds the same number of elements (C0 = WIDTH /
    // 256), so every merge combines two equal power-of-two counts and takes
    // welford_merge_equal's constant weights; and the four trees can share
    // registers once half of a tree's lanes are idle: each merge below pairs
    // the same two virtual lanes, in the same operand order, as the per-warp
    // tree.
    constexpr int C0 = WIDTH / 256;
    // Level 32 per virtual warp: lanes 0..31 of each hold its live states.
#pragma unroll
    for (int w = 0; w < 4; ++w) st[w] = welford_merge_equal<C0>(st[w], shfl_down_stats(st[w], 32));
    // Pack: p01 = warp 0 in lanes 0..31, warp 1 in lanes 32..63; p23 likewise.
    const bool upper32 = lane >= 32;
    Welford p01 = st[0], p23 = st[2];
    {
      const float m1 = __shfl_xor(st[1].mean, 32, kWave), q1 = __shfl_xor(st[1].m2, 32, kWave);
      const float m3 = __shfl_xor(st[3].mean, 32, kWave), q3 = __shfl_xor(st[3].m2, 32, kWave);
      if (upper32) {
        p01.mean = m1;
        p01.m2 = q1;
        p23.mean = m3;
        p23.m2 = q3;
      }
    }
    // Level 16 within each 32-lane half.
    p01 = welford_merge_equal<2 * C0>(p01, shfl_down_stats(p01, 16));
    p23 = welford_merge_equal<2 * C0>(p23, shfl_down_stats(p23, 16));
    // Pack: q = warp 0 | warp 2 | warp 1 | warp 3 in lanes 0..15 | 16..31 |
    // 32..47 | 48..63 (lanes with bit 4 set take p23 from lane ^ 16).
    Welford q = p01;
    {
      const float m = __shfl_xor(p23.mean, 16, kWave), q2 = __shfl_xor(p23.m2, 16, kWave);
      if (lane & 16) {
        q.mean = m;
        q.m2 = q2;
      }
    }
    // Levels 8..1 within each 16-lane group: lanes 0, 16, 32, 48 end with the
    // totals of warps 0, 2, 1, 3.
    q = welford_merge_equal<4 * C0>(q, shfl_down_stats(q, 8));
    q = welford_merge_equal<8 * C0>(q, shfl_down_stats(q, 4));
    q = welford_merge_equal<16 * C0>(q, shfl_down_stats(q, 2));
    q = welford_merge_equal<32 * C0>(q, shfl_down_stats(q, 1));
    // Cross-warp merges: (0 <- 2) at lane 0, (1 <- 3) at lane 32, then (0 <- 1).
    q = welford_merge_equal<64 * C0>(q, shfl_down_stats(q, 16));
    q = welford_merge_equal<128 * C0>(q, shfl_down_stats(q, 32));
    mean_all = q.mean;
    m2_all = q.m2;
  } else {
    // WIDTH 256 or 512: virtual threads 0 .. WIDTH/4 - 1 (virtual warps 0 and,
    // at 512, 1) hold one 4-element vector each and the others none.  Inside
    // a non-empty warp every merge combines two equal power-of-two counts
    // (welford_merge_equal); an empty warp's tree stays empty; and merging an
    // empty state into a state of 256 elements is an identity (weights
    // 0 * rcp(256) = 0 and 256 * rcp(256) = 1, both exact), so of the
    // cross-warp merges only (0 <- 1) at 512 changes anything.
    static_assert(WIDTH == 256 || WIDTH == 512, "one vector per virtual thread of warps 0 (and 1)");
    const bool upper32 = lane >= 32;
    st[0] = welford_merge_equal<4>(st[0], shfl_down_stats(st[0], 32));
    Welford q = st[0];
    if constexpr (WIDTH == 512) {
      // warp 1's level 32, then warp 0 in lanes 0..31 and warp 1 in 32..63
      st[1] = welford_merge_equal<4>(st[1], shfl_down_stats(st[1], 32));
      const float m1 = __shfl_xor(st[1].mean, 32, kWave), q1 = __shfl_xor(st[1].m2, 32, kWave);
      if (upper32) {
        q.mean = m1;
        q.m2 = q1;
      }
    }
    // levels 16..1 within each 32-lane half (lane 0: warp 0, lane 32: warp 1)
    q = welford_merge_equal<8>(q, shfl_down_stats(q, 16));
    q = welford_merge_equal<16>(q, shfl_down_stats(q, 8));
    q = welford_merge_equal<32>(q, shfl_down_stats(q, 4));
    q = welford_merge_equal<64>(q, shfl_down_stats(q, 2));
    q = welford_merge_equal<128>(q, shfl_down_stats(q, 1));
    if constexpr (WIDTH == 512) q = welford_merge_equal<256>(q, shfl_down_stats(q, 32));
    mean_all = q.mean;
    m2_all = q.m2;
  }
  const float mean = __shfl(mean_all, 0, kWave);
  const float var = __shfl(m2_all, 0, kWave) / static_cast<float>(WIDTH);
  const float rstd = rsqrtf(var + eps);

  if (!has) return;
  if constexpr (!kEarlyAffine) load_affine();
#pragma unroll
  for (int s = 0; s < kSlots; ++s) {
    const int base = (lane + kWave * s) * 4;
    const float g[4] = {lo_bf16(gw[s][0]), hi_bf16(gw[s][0]), lo_bf16(gw[s][1]), hi_bf16(gw[s][1])};
    const float b[4] = {lo_bf16(bw[s][0]), hi_bf16(bw[s][0]), lo_bf16(bw[s][1]), hi_bf16(bw[s][1])};
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = fmaf(g[e], rstd * (v[s][e] - mean), b[e]);
    *reinterpret_cast<u32x2*>(yr + base) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  }
}

// Rows narrower than 256 (L = WIDTH / 4 < 64 vectors): 64 / L rows share a
// wavefront, L lanes (one vector each) per row; packed_row_stats reproduces
// the reference's merges with the empty lanes of its 64-lane warp.
template <int WIDTH>
__global__ void __launch_bounds__(kRowsPerBlock * kWave)
layernorm_packed_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ gamma,
                        const bf16_t* __restrict__ beta, bf16_t* __restrict__ y, int64_t rows, float eps,
                        const uint8_t* __restrict__ row_mask) {
  constexpr int L = WIDTH / 4;   // lanes per row
  constexpr int R = kWave / L;   // rows per wavefront
  static_assert(L >= 8 && L <= 32, "packed widths 32..128");
  const int lane = threadIdx.x % kWave;
  const int seg = lane / L;      // this lane's row within the wavefront
  const int j = lane % L;        // this lane's vector within the row
  const int64_t row = (static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave) * R + seg;
  const bool live = row < rows;  // every lane stays for the shuffles
  const int64_t base = (live ? row : 0) * WIDTH + j * 4;

  const u32x2 w = *reinterpret_cast<const u32x2*>(x + base);
  const u32x2 gw = *reinterpret_cast<const u32x2*>(gamma + j * 4);
  const u32x2 bw = *reinterpret_cast<const u32x2*>(beta + j * 4);
  const float v[4] = {lo_bf16(w[0]), hi_bf16(w[0]), lo_bf16(w[1]), hi_bf16(w[1])};

  float mean, rstd;
  packed_row_stats<L>(v, j, seg, eps, &mean, &rstd);
  if (!live) return;

  u32x2 out = {0u, 0u};
  if (row_mask == nullptr || row_mask[row] != 0) {
    const float g[4] = {lo_bf16(gw[0]), hi_bf16(gw[0]), lo_bf16(gw[1]), hi_bf16(gw[1])};
    const float b[4] = {lo_bf16(bw[0]), hi_bf16(bw[0]), lo_bf16(bw[1]), hi_bf16(bw[1])};
    float o[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = fmaf(g[e], rstd * (v[e] - mean), b[e]);
    out = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
  }
  *reinterpret_cast<u32x2*>(y + base) = out;
}

template <int WIDTH>
hipError_t launch_ln(const bf16_t* x, const bf16_t* g, const bf16_t* b, bf16_t* y,
                     int64_t rows, float eps, const uint8_t* mask, hipStream_t st) {
  if constexpr (WIDTH < 256) {
    constexpr int kRowsPerWave = kWave / (WIDTH / 4);
    const int64_t per_block = static_cast<int64_t>(kRowsPerBlock) * kRowsPerWave;
    const int64_t blocks = (rows + per_block - 1) / per_block;
    hipLaunchKernelGGL(layernorm_packed_kernel<WIDTH>, dim3(static_cast<uint32_t>(blocks)),
                       dim3(kRowsPerBlock * kWave), 0, st, x, g, b, y, rows, eps, mask);
  } else {
    const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
    hipLaunchKernelGGL(layernorm_kernel<WIDTH>, dim3(static_cast<uint32_t>(blocks)),
                       dim3(kRowsPerBlock * kWave), 0, st, x, g, b, y, rows, eps, mask);
  }
  return hipGetLastError();
}

}  // namespace

bool layernorm_supported(int64_t width) {
  return width == 32 || width == 64 || width == 128 || width == 256 || width == 512 || width == 1024 ||
         width == 2048 || width == 4096;
}

hipError_t layernorm_bf16(const bf16_t* x, const bf16_t* gamma, const bf16_t* beta, bf16_t* y,
                          int64_t rows, int64_t width, float eps, const uint8_t* row_mask,
                          hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  switch (width) {
    case 32: return launch_ln<32>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 64: return launch_ln<64>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 128: return launch_ln<128>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 256: return launch_ln<256>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 512: return launch_ln<512>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 1024: return launch_ln<1024>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 2048: return launch_ln<2048>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 4096: return launch_ln<4096>(x, gamma, beta, y, rows, eps, row_mask, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace enc
