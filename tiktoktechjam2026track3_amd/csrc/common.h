// Shared device helpers for the gfx950 encoder kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

// Raw buffer load into LDS (the LLVM intrinsic, bound by name): byte address =
// resource base + soffset + voffset; the LDS destination is the instruction's
// uniform base (M0) plus `size` bytes per lane.
typedef int32_t enc_rsrc_t __attribute__((ext_vector_type(4)));
__device__ void enc_buffer_load_lds(enc_rsrc_t rsrc, __attribute__((address_space(3))) uint32_t* lds, int size,
                                    int voffset, int soffset, int offset, int aux)
    __asm("llvm.amdgcn.raw.buffer.load.lds");

namespace enc {

typedef uint16_t bf16_t;  // IEEE bfloat16 storage
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x16 __attribute__((ext_vector_type(16)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

constexpr int kWave = 64;

__device__ __forceinline__ float bf16_to_f32(bf16_t v) {
  return __uint_as_float(static_cast<uint32_t>(v) << 16);
}

// Round-to-nearest-even float -> bf16 (gfx950 v_cvt_pk_bf16_f32).
__device__ __forceinline__ bf16_t f32_to_bf16(float v) {
  __bf16 h = static_cast<__bf16>(v);
  return __builtin_bit_cast(bf16_t, h);
}

typedef float f32x2 __attribute__((ext_vector_type(2)));

// Two floats -> packed bf16 pair (lo in bits 0..15), round to nearest even.
// The vector conversion maps onto one v_cvt_pk_bf16_f32 for both values.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const f32x2 v = {lo, hi};
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
}

// Round a float to the nearest bf16 value and return it as float: one
// v_cvt_pk_bf16_f32 with bf16(0) = 0 in the low half and bf16(v) in the high
// half is exactly the fp32 encoding of bf16(v), so no unpacking follows.  The
// zero comes through an empty asm (one register per kernel after CSE): with a
// literal 0 the compiler rewrites the conversion into a convert to the low
// half plus a shift.  (The conversion itself must stay a compiler-visible
// instruction: as inline asm it could read an MFMA result before the MFMA
// has written it, since hazards around asm operands are not tracked.)
__device__ __forceinline__ float opaque_zero() {
  float z;
  asm("v_mov_b32 %0, 0" : "=v"(z));
  return z;
}
__device__ __forceinline__ float round_bf16(float v) {
  const f32x2 pair = {opaque_zero(), v};
  return __builtin_bit_cast(float, __builtin_convertvector(pair, bf16x2));
}

__device__ __forceinline__ float lo_bf16(uint32_t w) { return __uint_as_float(w << 16); }
__device__ __forceinline__ float hi_bf16(uint32_t w) { return __uint_as_float(w & 0xffff0000u); }

// expf(x) for x <= 0 (or -inf), bit for bit what the device library's expf
// returns: the same operation sequence (x * log2(e) split into a rounded
// product and an fma-recovered low part, nearest-integer split, v_exp_f32 of
// the fraction, ldexp by the integer part) and the same underflow clamp to 0
// below -103.28, without the overflow clamp, which cannot fire for x <= 0.
// Softmax exponentials exp(s - max) are its only use.
//
// expf_nonpos_unclamped is the same sequence without the underflow clamp, for
// callers that know x is finite and x >= -103.27893 (where the clamp returns
// the unclamped value): two VALU instructions fewer per call.
__device__ __forceinline__ float expf_nonpos_unclamped(float x) {
#pragma clang fp contract(off)
  const float l2e = __uint_as_float(0x3fb8aa3bu);     // log2(e) rounded
  const float l2e_lo = __uint_as_float(0x32a5705fu);  // log2(e) - l2e
  const float ph = x * l2e;
  float pl = __builtin_fmaf(x, l2e, -ph);
  pl = __builtin_fmaf(x, l2e_lo, pl);
  const float n = __builtin_rintf(ph);
  const float f = (ph - n) + pl;
  return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(f), static_cast<int>(n));
}
__device__ __forceinline__ float expf_nonpos(float x) {
  const float r = expf_nonpos_unclamped(x);
  return (x < __uint_as_float(0xc2ce8ed0u)) ? 0.f : r;  // -103.27893
}

// expf_nonpos(g * s) for a power-of-two s, without forming g * s: s is folded
// into the two log2(e) constants (s * l2e and s * l2e_lo are exact), so the
// rounded product x * l2e and both fma's see the same exact real values as
// with x = g * s, and return the same bits.  (g * s itself is exact for the
// softmax gaps, differences of two bf16 values, even as a subnormal: their
// spacing is at least 2^-133.)  Callers pass the folded constants
// (expf_scaled_consts) and the clamp bound -103.27893 / s.
struct ExpfScaled {
  float l2e, l2e_lo, clamp;
};
__device__ __forceinline__ ExpfScaled expf_scaled_consts(float s) {
  return ExpfScaled{__uint_as_float(0x3fb8aa3bu) * s, __uint_as_float(0x32a5705fu) * s,
                    __uint_as_float(0xc2ce8ed0u) / s};
}
__device__ __forceinline__ float expf_nonpos_scaled_unclamped(float g, const ExpfScaled& c) {
#pragma clang fp contract(off)
  const float ph = g * c.l2e;
  float pl = __builtin_fmaf(g, c.l2e, -ph);
  pl = __builtin_fmaf(g, c.l2e_lo, pl);
  const float n = __builtin_rintf(ph);
  const float f = (ph - n) + pl;
  return __builtin_amdgcn_ldexpf(__builtin_amdgcn_exp2f(f), static_cast<int>(n));
}
__device__ __forceinline__ float expf_nonpos_scaled(float g, const ExpfScaled& c) {
  const float r = expf_nonpos_scaled_unclamped(g, c);
  return (g < c.clamp) ? 0.f : r;
}

// Exact-erf GELU in fp32: 0.5 * x * (1 + erf(x / sqrt(2))).
__device__ __forceinline__ float gelu_erf(float x) {
  return 0.5f * x * (1.0f + erff(x * 0.70710678118654752440f));
}

// s_waitcnt immediate (gfx9 encoding): wait until at most `vm` vector-memory
// and `lgkm` LDS operations of this wavefront are outstanding.
constexpr int waitcnt_imm(int vm, int lgkm) {
  return (vm & 15) | ((vm >> 4) << 14) | (7 << 4) | ((lgkm & 15) << 8);
}

// Workgroup barrier for global->LDS rings.  __syncthreads() is also a
// workgroup release/acquire fence, which the compiler implements with
// s_waitcnt vmcnt(0): that drains every prefetched stage still in flight.
// Here the caller first waits (s_waitcnt) for exactly the loads and LDS reads
// it needs finished; the memory clobber keeps the compiler from moving LDS
// accesses across the barrier.
__device__ __forceinline__ void ring_barrier() { asm volatile("s_barrier" ::: "memory"); }

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));
// Buffer resource over [p, p + 4 GiB): stride 0, no range limit, the gfx9
// raw-buffer format word.  Callers keep every load inside their own rows.
__device__ __forceinline__ i32x4 buffer_rsrc(const void* p) {
  const uint64_t a = reinterpret_cast<uint64_t>(p);
  return i32x4{static_cast<int32_t>(static_cast<uint32_t>(a)),
               static_cast<int32_t>(static_cast<uint32_t>(a >> 32) & 0xffffu), -1, 0x00020000};
}

// LDS address of a pointer into a __shared__ array, as the buffer-to-LDS load
// takes it (the low 32 bits of the flat address are the LDS offset).
__device__ __forceinline__ __attribute__((address_space(3))) uint32_t* lds_ptr(const void* p) {
  return reinterpret_cast<__attribute__((address_space(3))) uint32_t*>(reinterpret_cast<uintptr_t>(p));
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, kWave);
  return v;
}

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) v = fmaxf(v, __shfl_xor(v, off, kWave));
  return v;
}

}  // namespace enc
