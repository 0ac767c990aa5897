// Shared device helpers for the HS-Guard MI355X kernels (gfx950, wave64).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/hsg.h"

namespace hsg {

// 16-byte register vectors are native clang vectors: a HIP uint4 / float4 copied whole is a struct memcpy that
// the compiler may not keep in registers (it parked such a buffer in LDS, and in another kernel in scratch)
typedef __attribute__((ext_vector_type(4))) uint32_t u32x4;

// ---- bf16 / fp16 scalar conversions (bf16 stored as uint16_t; round to nearest even like torch) ----
__device__ __forceinline__ float bf2f(uint16_t h) { return __uint_as_float(((uint32_t)h) << 16); }

__device__ __forceinline__ uint16_t f2bf(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);
  return (uint16_t)(u >> 16);
}

__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// round-to-nearest-even fp32 -> bf16 without the NaN case (callers pass finite values), branch-free
__device__ __forceinline__ uint16_t f2bf_finite(float f) {
  const uint32_t u = __float_as_uint(f);
  return (uint16_t)((u + 0x7fffu + ((u >> 16) & 1u)) >> 16);
}

// two finite fp32 values -> packed bf16 pair (a in the low half), round to nearest even: one v_cvt_pk_bf16_f32
typedef __attribute__((ext_vector_type(2))) float f32x2_;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_;
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_){a, b}, bf16x2_));
}

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// ---- vector loads of bf16 (addresses must be 16 / 8 byte aligned; the C-ABI checks) ----
__device__ __forceinline__ void unpack2(uint32_t w, float& lo, float& hi) {
  lo = __uint_as_float(w << 16);
  hi = __uint_as_float(w & 0xffff0000u);
}

__device__ __forceinline__ void load8_bf16(const uint16_t* p, float* x) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  unpack2(w.x, x[0], x[1]);
  unpack2(w.y, x[2], x[3]);
  unpack2(w.z, x[4], x[5]);
  unpack2(w.w, x[6], x[7]);
}

__device__ __forceinline__ void load4_bf16(const uint16_t* p, float* x) {
  const uint2 w = *reinterpret_cast<const uint2*>(p);
  unpack2(w.x, x[0], x[1]);
  unpack2(w.y, x[2], x[3]);
}

__device__ __forceinline__ void store4_bf16(uint16_t* p, const float* x) {
  uint2 w;
  w.x = (uint32_t)f2bf(x[0]) | ((uint32_t)f2bf(x[1]) << 16);
  w.y = (uint32_t)f2bf(x[2]) | ((uint32_t)f2bf(x[3]) << 16);
  *reinterpret_cast<uint2*>(p) = w;
}

__device__ __forceinline__ float sigmoidf_(float x) { return 1.0f / (1.0f + expf(-x)); }
__device__ __forceinline__ float siluf_(float x) { return x / (1.0f + expf(-x)); }

// ---- wave64 butterfly sums (every lane ends with the same bitwise value) ----
template <int MASK>
__device__ __forceinline__ float xor_add(float x) { return x + __shfl_xor(x, MASK, 64); }

template <int MASK>
__device__ __forceinline__ float xor_max(float x) { return fmaxf(x, __shfl_xor(x, MASK, 64)); }

__device__ __forceinline__ float wave_sum(float x) {
  x = xor_add<1>(x); x = xor_add<2>(x); x = xor_add<4>(x);
  x = xor_add<8>(x); x = xor_add<16>(x); x = xor_add<32>(x);
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  x = xor_max<1>(x); x = xor_max<2>(x); x = xor_max<4>(x);
  x = xor_max<8>(x); x = xor_max<16>(x); x = xor_max<32>(x);
  return x;
}

inline bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? HSG_OK : (int)e;
}

}  // namespace hsg
