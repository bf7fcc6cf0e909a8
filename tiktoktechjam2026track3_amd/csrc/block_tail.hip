// Fused block tail for narrow encoders (d_model and ffn_dim of 32, 64 or 128).
//
// After the attention, the reference's block runs (models.py:733-737)
//   x_attn = x + out_proj(context)          rows masked out keep x
//   h      = gelu(ffn_in(norm2(x_attn)))
//   x_out  = x_attn + ffn_out(h)            rows masked out become 0
// which the wide path launches as four kernels with [T, D] / [T, F] round
// trips through memory.  With d_model and ffn_dim <= 128 the three weight
// matrices fit in LDS together (104 KB at 128 / 128), so one persistent
// workgroup per CU loads them once and walks 16-row slabs of the tokens: the
// context and residual rows come in, every intermediate stays in LDS, and
// only x_out goes out (with, optionally, the next layer's norm1 of the same
// rows).  For these sizes the products are latency-bound and the launches it
// saves per layer (three, four with the next norm1) matter more than MFMA
// rate.
//
// The arithmetic is the wide path's, operation for operation, so the output
// is bitwise the same: each product accumulates K sequentially in 16-deep
// MFMA steps (v_mfma_f32_16x16x16_bf16, as the skinny GEMM; the library splits
// none of these shapes), y = bf16(acc + bias) at the nn.Linear boundary, the
// residual adds and GELU-erf as in the GEMM epilogues, and norm2 through
// packed_row_stats, the LayerNorm kernel's reduction for rows of <= 128.
#include "common.h"
#include "kernels.h"
#include "welford.h"

namespace enc {

namespace {

constexpr int kTailRows = 16;       // rows per slab: the MFMA M dimension
constexpr int kTailThreads = 256;  // 4 wavefronts

typedef short s16x4 __attribute__((ext_vector_type(4)));

// LDS row stride of a K-wide operand, bf16 elements: 16 bytes of padding put
// consecutive rows 4 banks apart, so the 16 rows of a fragment read spread
// over all 64 banks.
constexpr int tail_ld(int k) { return k + 8; }

// LDS layout, bf16 elements: Wo [D][D], W1 [F][D], W2 [D][F], then slab
// buffers A [16][D] (context, then norm2 output, then the block output), X
// [16][D] (residual, then x_attn) and Hd [16][F] (GELU output), each row
// padded to tail_ld.
constexpr size_t tail_lds_bytes(int d, int f) {
  return 2 * (static_cast<size_t>(d) * tail_ld(d) + static_cast<size_t>(f) * tail_ld(d) +
              static_cast<size_t>(d) * tail_ld(f) + kTailRows * (2 * static_cast<size_t>(tail_ld(d)) + tail_ld(f)));
}

// MFMA fragment of LDS row `row` (K-wide operand) at K offset k0: lane group g
// holds k0 + 4g .. k0 + 4g + 3 (A: row = l % 16; B: row = output column).
template <int K>
__device__ __forceinline__ s16x4 tail_frag(const bf16_t* base, int row, int k0, int g) {
  return *reinterpret_cast<const s16x4*>(base + row * tail_ld(K) + k0 + 4 * g);
}

// NROWS x K bf16 row-major (global) <-> registers <-> LDS (padded stride):
// chunk i of this thread is 16-byte chunk tid + 256 i of the matrix.  The
// three weight matrices are loaded into registers together and only then
// stored, so their loads share one memory round trip.
template <int K, int NROWS>
struct TailRows {
  static constexpr int kChunks = K / 8;
  static constexpr int kTotal = NROWS * kChunks;
  static constexpr int kPer = (kTotal + kTailThreads - 1) / kTailThreads;  // chunks per thread
  __device__ static void load(u32x4 (&v)[kPer], const bf16_t* src, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = min(tid + i * kTailThreads, kTotal - 1);
      v[i] = *reinterpret_cast<const u32x4*>(src + static_cast<int64_t>(c / kChunks) * K + (c % kChunks) * 8);
    }
  }
  __device__ static void store(const u32x4 (&v)[kPer], bf16_t* dst, int tid) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = tid + i * kTailThreads;
      if (kTotal % kTailThreads == 0 || c < kTotal)
        *reinterpret_cast<u32x4*>(dst + (c / kChunks) * tail_ld(K) + (c % kChunks) * 8) = v[i];
    }
  }
};

template <int D, int F>
__global__ void __launch_bounds__(kTailThreads)
block_tail_kernel(const bf16_t* __restrict__ ctx, const bf16_t* __restrict__ x, const bf16_t* __restrict__ wo,
                  const bf16_t* __restrict__ bo, const bf16_t* __restrict__ g2, const bf16_t* __restrict__ be2,
                  const bf16_t* __restrict__ w1, const bf16_t* __restrict__ b1, const bf16_t* __restrict__ w2,
                  const bf16_t* __restrict__ b2, bf16_t* __restrict__ out, int rows, float eps,
                  const uint8_t* __restrict__ row_mask, const bf16_t* __restrict__ g1n,
                  const bf16_t* __restrict__ be1n, bf16_t* __restrict__ ln_out) {
  static_assert((D == 32 || D == 64 || D == 128) && (F == 32 || F == 64 || F == 128), "d_model, ffn_dim");
  constexpr int kLdD = tail_ld(D), kLdF = tail_ld(F);
  constexpr int kSlabChunks = kTailRows * (D / 8);  // 16-byte chunks of a [16][D] slab
  static_assert(kSlabChunks <= kTailThreads, "one chunk of each slab operand per thread");
  extern __shared__ __attribute__((aligned(16))) bf16_t tail_lds[];
  bf16_t* sWo = tail_lds;
  bf16_t* sW1 = sWo + D * kLdD;
  bf16_t* sW2 = sW1 + F * kLdD;
  bf16_t* sA = sW2 + D * kLdF;
  bf16_t* sX = sA + kTailRows * kLdD;
  bf16_t* sH = sX + kTailRows * kLdD;

  const int tid = threadIdx.x;
  const int lane = tid % kWave;
  const int wave = __builtin_amdgcn_readfirstlane(tid / kWave);
  const int l16 = lane & 15;
  const int g = lane >> 4;

  {
    using RWo = TailRows<D, D>;
    using RW1 = TailRows<D, F>;
    using RW2 = TailRows<F, D>;
    u32x4 vo[RWo::kPer], v1[RW1::kPer], v2[RW2::kPer];
    RWo::load(vo, wo, tid);
    RW1::load(v1, w1, tid);
    RW2::load(v2, w2, tid);
    RWo::store(vo, sWo, tid);
    RW1::store(v1, sW1, tid);
    RW2::store(v2, sW2, tid);
  }

  // norm2's gamma / beta for this lane's vector (rows of D = 4 L elements)
  constexpr int L = D / 4;
  constexpr int R = kWave / L;  // rows per wavefront in the norm2 pass
  const int seg = lane / L, j = lane % L;
  const u32x2 gw = *reinterpret_cast<const u32x2*>(g2 + 4 * j);
  const u32x2 bw = *reinterpret_cast<const u32x2*>(be2 + 4 * j);
  // the next layer's norm1 (optional: ln_out == nullptr skips it)
  const bool next_norm = ln_out != nullptr;
  u32x2 gn = {0u, 0u}, bn = {0u, 0u};
  if (next_norm) {
    gn = *reinterpret_cast<const u32x2*>(g1n + 4 * j);
    bn = *reinterpret_cast<const u32x2*>(be1n + 4 * j);
  }

  // the slab's context and residual chunks travel in registers one slab ahead
  const int slabs = (rows + kTailRows - 1) / kTailRows;
  const int my_r = tid / (D / 8), my_ch = tid % (D / 8);
  const bool has_chunk = tid < kSlabChunks;
  u32x4 next_a = {0u, 0u, 0u, 0u}, next_x = {0u, 0u, 0u, 0u};
  auto fetch = [&](int slab) {
    next_a = u32x4{0u, 0u, 0u, 0u};
    next_x = u32x4{0u, 0u, 0u, 0u};
    const int r = slab * kTailRows + my_r;
    if (has_chunk && slab < slabs && r < rows) {
      next_a = *reinterpret_cast<const u32x4*>(ctx + static_cast<int64_t>(r) * D + my_ch * 8);
      next_x = *reinterpret_cast<const u32x4*>(x + static_cast<int64_t>(r) * D + my_ch * 8);
    }
  };
  fetch(blockIdx.x);

  for (int slab = blockIdx.x; slab < slabs; slab += gridDim.x) {
    const int r0 = slab * kTailRows;
    __syncthreads();  // the previous slab's output copy has read sA (and the weights have landed)
    if (has_chunk) {
      *reinterpret_cast<u32x4*>(sA + my_r * kLdD + my_ch * 8) = next_a;
      *reinterpret_cast<u32x4*>(sX + my_r * kLdD + my_ch * 8) = next_x;
    }
    fetch(slab + gridDim.x);
    // Row-mask verdicts of this lane's output rows 4g .. 4g+3, taken before
    // the products: with no branch between an MFMA and the reads of its
    // result, the compiler's wait states before those reads stay in place
    // (a mask test between them left a result register read two
    // instructions after its MFMA, before the write landed).
    bool keep[4];
#pragma unroll
    for (int jj = 0; jj < 4; ++jj) {
      const int r = r0 + 4 * g + jj;
      keep[jj] = row_mask == nullptr || (r < rows && row_mask[r] != 0);
    }
    __syncthreads();

    // ---- out_proj + residual (rows masked out keep the residual) -> sX ----
    for (int cb = wave; cb < D / 16; cb += 4) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(tail_frag<D>(sA, l16, ks * 16, g),
                                                        tail_frag<D>(sWo, cb * 16 + l16, ks * 16, g), acc, 0, 0, 0);
      const int col = cb * 16 + l16;
      const float bias = bf16_to_f32(bo[col]);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int r = 4 * g + jj;
        const float y = round_bf16(acc[jj] + bias);  // nn.Linear output boundary
        bf16_t* px = sX + r * kLdD + col;
        const bf16_t old = *px;
        *px = keep[jj] ? f32_to_bf16(bf16_to_f32(old) + y) : old;
      }
    }
    __syncthreads();

    // ---- norm2 (no row mask) -> sA ----
    for (int p = 0; p < kTailRows; p += 4 * R) {
      const int r = p + wave * R + seg;
      const int rr = r < kTailRows ? r : kTailRows - 1;  // lanes past the slab only join the shuffles
      const u32x2 w = *reinterpret_cast<const u32x2*>(sX + rr * kLdD + 4 * j);
      const float v[4] = {lo_bf16(w[0]), hi_bf16(w[0]), lo_bf16(w[1]), hi_bf16(w[1])};
      float mean, rstd;
      packed_row_stats<L>(v, j, seg, eps, &mean, &rstd);
      if (r < kTailRows) {
        const float ga[4] = {lo_bf16(gw[0]), hi_bf16(gw[0]), lo_bf16(gw[1]), hi_bf16(gw[1])};
        const float be[4] = {lo_bf16(bw[0]), hi_bf16(bw[0]), lo_bf16(bw[1]), hi_bf16(bw[1])};
        float o[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) o[e] = fmaf(ga[e], rstd * (v[e] - mean), be[e]);
        *reinterpret_cast<u32x2*>(sA + r * kLdD + 4 * j) = u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
      }
    }
    __syncthreads();

    // ---- ffn_in + GELU -> sH ----
    for (int cb = wave; cb < F / 16; cb += 4) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < D / 16; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(tail_frag<D>(sA, l16, ks * 16, g),
                                                        tail_frag<D>(sW1, cb * 16 + l16, ks * 16, g), acc, 0, 0, 0);
      const int col = cb * 16 + l16;
      const float bias = bf16_to_f32(b1[col]);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const float y = round_bf16(acc[jj] + bias);
        sH[(4 * g + jj) * kLdF + col] = f32_to_bf16(gelu_erf(y));
      }
    }
    __syncthreads();

    // ---- ffn_out + residual (rows masked out become 0) -> sA ----
    for (int cb = wave; cb < D / 16; cb += 4) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < F / 16; ++ks)
        acc = __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(tail_frag<F>(sH, l16, ks * 16, g),
                                                        tail_frag<F>(sW2, cb * 16 + l16, ks * 16, g), acc, 0, 0, 0);
      const int col = cb * 16 + l16;
      const float bias = bf16_to_f32(b2[col]);
#pragma unroll
      for (int jj = 0; jj < 4; ++jj) {
        const int r = 4 * g + jj;
        const float y = round_bf16(acc[jj] + bias);
        sA[r * kLdD + col] = keep[jj] ? f32_to_bf16(bf16_to_f32(sX[r * kLdD + col]) + y) : bf16_t(0);
      }
    }
    __syncthreads();

    // ---- block output, 16-byte stores ----
    if (has_chunk && r0 + my_r < rows)
      *reinterpret_cast<u32x4*>(out + static_cast<int64_t>(r0 + my_r) * D + my_ch * 8) =
          *reinterpret_cast<const u32x4*>(sA + my_r * kLdD + my_ch * 8);

    // ---- the next layer's norm1 of the block output rows (no row mask, as
    // the separate launch) -> ln_out ----
    if (next_norm) {
      for (int p = 0; p < kTailRows; p += 4 * R) {
        const int r = p + wave * R + seg;
        const int rr = r < kTailRows ? r : kTailRows - 1;  // lanes past the slab only join the shuffles
        const u32x2 w = *reinterpret_cast<const u32x2*>(sA + rr * kLdD + 4 * j);
        const float v[4] = {lo_bf16(w[0]), hi_bf16(w[0]), lo_bf16(w[1]), hi_bf16(w[1])};
        float mean, rstd;
        packed_row_stats<L>(v, j, seg, eps, &mean, &rstd);
        if (r < kTailRows && r0 + r < rows) {
          const float ga[4] = {lo_bf16(gn[0]), hi_bf16(gn[0]), lo_bf16(gn[1]), hi_bf16(gn[1])};
          const float be[4] = {lo_bf16(bn[0]), hi_bf16(bn[0]), lo_bf16(bn[1]), hi_bf16(bn[1])};
          float o[4];
#pragma unroll
          for (int e = 0; e < 4; ++e) o[e] = fmaf(ga[e], rstd * (v[e] - mean), be[e]);
          *reinterpret_cast<u32x2*>(ln_out + static_cast<int64_t>(r0 + r) * D + 4 * j) =
              u32x2{pack_bf16x2(o[0], o[1]), pack_bf16x2(o[2], o[3])};
        }
      }
    }
  }
}

template <int D, int F>
hipError_t launch_tail(const BlockTailArgs& a, int rows, float eps, int num_cus, hipStream_t st) {
  auto kernel = block_tail_kernel<D, F>;
  constexpr size_t kLds = tail_lds_bytes(D, F);
  if constexpr (kLds > 64 * 1024) {
    // above 64 KiB of dynamic LDS the kernel has to opt in (once per process)
    static const hipError_t attr = hipFuncSetAttribute(reinterpret_cast<const void*>(kernel),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       static_cast<int>(kLds));
    if (attr != hipSuccess) return attr;
  }
  const int slabs = (rows + kTailRows - 1) / kTailRows;
  const int grid = slabs < num_cus ? slabs : num_cus;
  hipLaunchKernelGGL(kernel, dim3(grid), dim3(kTailThreads), kLds, st, a.ctx, a.x, a.wo, a.bo, a.g2, a.be2, a.w1,
                     a.b1, a.w2, a.b2, a.out, rows, eps, a.row_mask, a.g1n, a.be1n, a.ln_out);
  return hipGetLastError();
}

template <int D>
hipError_t launch_tail_f(int f, const BlockTailArgs& a, int rows, float eps, int num_cus, hipStream_t st) {
  switch (f) {
    case 32: return launch_tail<D, 32>(a, rows, eps, num_cus, st);
    case 64: return launch_tail<D, 64>(a, rows, eps, num_cus, st);
    case 128: return launch_tail<D, 128>(a, rows, eps, num_cus, st);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

bool block_tail_supported(int64_t d_model, int64_t ffn_dim) {
  auto ok = [](int64_t v) { return v == 32 || v == 64 || v == 128; };
  return ok(d_model) && ok(ffn_dim);
}

hipError_t block_tail_bf16(const BlockTailArgs& a, int64_t rows, int64_t d_model, int64_t ffn_dim, float eps,
                           int num_cus, hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  if (!block_tail_supported(d_model, ffn_dim) || rows >= (int64_t(1) << 31)) return hipErrorInvalidValue;
  // the kernel reads x and writes out through restrict pointers
  if (a.out == a.x || (a.ln_out != nullptr && (a.ln_out == a.x || a.ln_out == a.out))) return hipErrorInvalidValue;
  const int r = static_cast<int>(rows);
  switch (d_model) {
    case 32: return launch_tail_f<32>(static_cast<int>(ffn_dim), a, r, eps, num_cus, stream);
    case 64: return launch_tail_f<64>(static_cast<int>(ffn_dim), a, r, eps, num_cus, stream);
    case 128: return launch_tail_f<128>(static_cast<int>(ffn_dim), a, r, eps, num_cus, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace enc
