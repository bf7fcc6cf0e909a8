// Welford statistics of torch's ROCm LayerNorm (vectorised kernel), shared by
// the LayerNorm kernels and the fused block tail.  The operation order is the
// reference's: per virtual thread, Welford updates of its 4-element vectors;
// per 64-lane virtual warp, a shuffle-down tree of the Welford combine; then
// the warps 0+2, 1+3, 0+1.
#pragma once

#include "common.h"

namespace enc {

struct Welford {
  float mean, m2, count;
};

// v_rcp_f32 of a value the compiler may know; the asm keeps it from folding.
__device__ __forceinline__ float hw_rcp(float n) {
  float r;
  asm("v_rcp_f32 %0, %1" : "=v"(r) : "v"(n));
  return r;
}

__device__ __forceinline__ Welford welford_add(Welford s, float x) {
#pragma clang fp contract(off)
  const float delta = x - s.mean;
  const float n = s.count + 1.f;
  const float mean = fmaf(delta, hw_rcp(n), s.mean);
  const float m2 = s.m2 + delta * (x - mean);
  return {mean, m2, n};
}

// combine(b = running, a = incoming), the operand roles of the native merge.
__device__ __forceinline__ Welford welford_merge(Welford b, Welford a) {
#pragma clang fp contract(off)
  const float delta = b.mean - a.mean;
  const float n = a.count + b.count;
  if (!(n > 0.f)) return {0.f, 0.f, n};
  const float coef = hw_rcp(n);
  const float na = a.count * coef;
  const float nb = b.count * coef;
  const float mean = na * a.mean + nb * b.mean;
  const float m2 = fmaf(delta * delta * a.count, nb, a.m2 + b.m2);
  return {mean, m2, n};
}

// welford_merge of two states that both hold C elements, C a power of two
// (every merge of a row whose virtual threads all hold the same count): the
// weights a.count * rcp(2C) and b.count * rcp(2C) are exactly 0.5 (v_rcp_f32
// of a power of two is exact), so they are constants, and the same rounded
// operations remain: mean = 0.5 a.mean + 0.5 b.mean, m2 = fma(delta^2 C,
// 0.5, a.m2 + b.m2).
template <int C>
__device__ __forceinline__ Welford welford_merge_equal(Welford b, Welford a) {
#pragma clang fp contract(off)
  static_assert(C > 0 && (C & (C - 1)) == 0, "equal power-of-two counts");
  const float delta = b.mean - a.mean;
  const float mean = 0.5f * a.mean + 0.5f * b.mean;
  const float m2 = fmaf(delta * delta * static_cast<float>(C), 0.5f, a.m2 + b.m2);
  return {mean, m2, static_cast<float>(2 * C)};
}

// mean and m2 only: the count is known to both sides
__device__ __forceinline__ Welford shfl_down_stats(Welford s, int off) {
  return {__shfl_down(s.mean, off, kWave), __shfl_down(s.m2, off, kWave), s.count};
}

__device__ __forceinline__ Welford shfl_down(Welford s, int off) {
  return {__shfl_down(s.mean, off, kWave), __shfl_down(s.m2, off, kWave),
          __shfl_down(s.count, off, kWave)};
}

// Statistics of a row of WIDTH = 4 L elements (L < 64) held one 4-element
// vector per lane: lanes seg*L .. seg*L + L - 1 of the wavefront hold row
// `seg`, lane seg*L + j its vector j.  The reference reduces such a row on a
// 64-lane warp whose lanes >= L hold empty (count 0) states, and merging an
// empty state is not an identity (the merge weights come from the hardware
// reciprocal of the count), so those merges are reproduced: at shuffle
// offsets >= L every lane merges an empty state, and below L a lane whose
// partner lies past its row's L lanes merges an empty state instead of the
// shuffled one (lane 0 of a row never reads another row's lanes).  The other
// virtual warps are empty: their merges follow as (w0 <- E) <- (E <- E).
// Every lane of the wavefront must call it (the shuffles span all lanes).
template <int L>
__device__ __forceinline__ void packed_row_stats(const float (&v)[4], int j, int seg, float eps, float* mean,
                                                 float* rstd) {
  static_assert(L >= 8 && L <= 32, "rows of 32..128 elements");
  Welford st = {0.f, 0.f, 0.f};
#pragma unroll
  for (int e = 0; e < 4; ++e) st = welford_add(st, v[e]);
  const Welford empty = {0.f, 0.f, 0.f};
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    if (off >= L) {
      st = welford_merge(st, empty);
    } else {
      Welford p = shfl_down(st, off);
      if (j + off >= L) p = empty;
      st = welford_merge(st, p);
    }
  }
  st = welford_merge(welford_merge(st, empty), welford_merge(empty, empty));
  *mean = __shfl(st.mean, seg * L, kWave);
  const float var = __shfl(st.m2, seg * L, kWave) / static_cast<float>(4 * L);
  *rstd = rsqrtf(var + eps);
}

}  // namespace enc
