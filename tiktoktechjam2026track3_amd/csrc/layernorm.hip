// Wavefront LayerNorm for bf16 activations (HBM-bound).
//
// One 64-lane wavefront owns one row of `width` elements; each lane keeps
// width/64 values in registers, so the row is read once and written once.
// Statistics are fp32 and two-pass over registers (mean, then the mean of the
// squared deviations), matching nn.LayerNorm's biased variance.  The output is
// gamma * ((x - mean) * rstd) + beta rounded once to bf16, the order used by
// the reference kernel (case6_exact_layer_norm.cu:118-128) and by ATen.
#include "common.h"
#include "kernels.h"

namespace enc {

namespace {

constexpr int kRowsPerBlock = 4;  // one row per wavefront, 4 wavefronts

// Element index owned by lane `lane`, slot `i` of VPT.
template <int VPT>
__device__ __forceinline__ int ln_index(int lane, int i) {
  if constexpr (VPT >= 8) {
    return (i / 8) * (kWave * 8) + lane * 8 + (i % 8);
  } else {
    return lane * VPT + i;
  }
}

template <int VPT>
__global__ void __launch_bounds__(kRowsPerBlock * kWave)
layernorm_kernel(const bf16_t* __restrict__ x, const bf16_t* __restrict__ gamma,
                 const bf16_t* __restrict__ beta, bf16_t* __restrict__ y,
                 int64_t rows, float eps, const uint8_t* __restrict__ row_mask) {
  constexpr int kWidth = VPT * kWave;
  const int lane = threadIdx.x % kWave;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const bf16_t* xr = x + row * kWidth;
  bf16_t* yr = y + row * kWidth;

  if (row_mask != nullptr && row_mask[row] == 0) {
    if constexpr (VPT >= 8) {
#pragma unroll
      for (int c = 0; c < VPT / 8; ++c)
        *reinterpret_cast<u32x4*>(yr + c * kWave * 8 + lane * 8) = u32x4{0, 0, 0, 0};
    } else {
#pragma unroll
      for (int i = 0; i < VPT; ++i) yr[lane * VPT + i] = 0;
    }
    return;
  }

  float v[VPT];
  if constexpr (VPT >= 8) {
#pragma unroll
    for (int c = 0; c < VPT / 8; ++c) {
      u32x4 w = *reinterpret_cast<const u32x4*>(xr + c * kWave * 8 + lane * 8);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        v[c * 8 + 2 * e] = lo_bf16(w[e]);
        v[c * 8 + 2 * e + 1] = hi_bf16(w[e]);
      }
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) v[i] = bf16_to_f32(xr[lane * VPT + i]);
  }

  float s = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) s += v[i];
  const float mean = wave_sum(s) * (1.0f / kWidth);
  float q = 0.f;
#pragma unroll
  for (int i = 0; i < VPT; ++i) {
    const float d = v[i] - mean;
    q += d * d;
  }
  const float var = wave_sum(q) * (1.0f / kWidth);
  const float rstd = rsqrtf(var + eps);

  if constexpr (VPT >= 8) {
#pragma unroll
    for (int c = 0; c < VPT / 8; ++c) {
      const int base = c * kWave * 8 + lane * 8;
      u32x4 gw = *reinterpret_cast<const u32x4*>(gamma + base);
      u32x4 bw = *reinterpret_cast<const u32x4*>(beta + base);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float y0 = lo_bf16(gw[e]) * ((v[c * 8 + 2 * e] - mean) * rstd) + lo_bf16(bw[e]);
        const float y1 = hi_bf16(gw[e]) * ((v[c * 8 + 2 * e + 1] - mean) * rstd) + hi_bf16(bw[e]);
        o[e] = pack_bf16x2(y0, y1);
      }
      *reinterpret_cast<u32x4*>(yr + base) = o;
    }
  } else {
#pragma unroll
    for (int i = 0; i < VPT; ++i) {
      const int idx = lane * VPT + i;
      const float out = bf16_to_f32(gamma[idx]) * ((v[i] - mean) * rstd) + bf16_to_f32(beta[idx]);
      yr[idx] = f32_to_bf16(out);
    }
  }
}

template <int VPT>
hipError_t launch_ln(const bf16_t* x, const bf16_t* g, const bf16_t* b, bf16_t* y,
                     int64_t rows, float eps, const uint8_t* mask, hipStream_t st) {
  const int64_t blocks = (rows + kRowsPerBlock - 1) / kRowsPerBlock;
  hipLaunchKernelGGL(layernorm_kernel<VPT>, dim3(static_cast<uint32_t>(blocks)),
                     dim3(kRowsPerBlock * kWave), 0, st, x, g, b, y, rows, eps, mask);
  return hipGetLastError();
}

}  // namespace

bool layernorm_supported(int64_t width) {
  return width == 64 || width == 128 || width == 256 || width == 512 || width == 1024 ||
         width == 2048 || width == 4096;
}

hipError_t layernorm_bf16(const bf16_t* x, const bf16_t* gamma, const bf16_t* beta, bf16_t* y,
                          int64_t rows, int64_t width, float eps, const uint8_t* row_mask,
                          hipStream_t stream) {
  if (rows == 0) return hipSuccess;
  switch (width) {
    case 64: return launch_ln<1>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 128: return launch_ln<2>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 256: return launch_ln<4>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 512: return launch_ln<8>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 1024: return launch_ln<16>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 2048: return launch_ln<32>(x, gamma, beta, y, rows, eps, row_mask, stream);
    case 4096: return launch_ln<64>(x, gamma, beta, y, rows, eps, row_mask, stream);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace enc
