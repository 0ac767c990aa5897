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

// two fp32 values -> packed bf16 pair (a in the low half), round to nearest even like torch: one
// v_cvt_pk_bf16_f32 (a NaN stays a NaN)
typedef __attribute__((ext_vector_type(2))) float f32x2_;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_;
__device__ __forceinline__ uint32_t pack_bf16x2(float a, float b) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_){a, b}, bf16x2_));
}

// fp32 -> bf16 on the same hardware conversion (branch-free)
__device__ __forceinline__ uint16_t f2bf(float f) { return (uint16_t)pack_bf16x2(f, f); }

__device__ __forceinline__ float rbf(float f) { return bf2f(f2bf(f)); }

// the same for values known to be finite (kept for call sites that state it)
__device__ __forceinline__ uint16_t f2bf_finite(float f) { return f2bf(f); }

__device__ __forceinline__ float h2f(uint16_t h) { return (float)__builtin_bit_cast(_Float16, h); }
__device__ __forceinline__ uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// ---- streaming loads of data read once per step (ring keys and values): the non-temporal hint, which on
// MI355X measured faster for these reads than ordinary loads (fused ring decode 142.0 -> 135.6 us at
// 352 x 1 on full rings) ----
typedef __attribute__((ext_vector_type(2))) uint32_t u32x2;
__device__ __forceinline__ uint4 ld_stream16(const uint16_t* p) {
  return __builtin_bit_cast(uint4, __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p)));
}
__device__ __forceinline__ uint2 ld_stream8(const uint16_t* p) {
  return __builtin_bit_cast(uint2, __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p)));
}

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

// ---- lane exchanges without the LDS crossbar: DPP modifiers (folded into the add) and gfx950's
// v_permlane16/32_swap. Each partial sum is a + b with a, b the two partners' values, so every lane of a
// group ends with the same bitwise value, as with the xor butterflies above. ----
template <int CTRL>
__device__ __forceinline__ float dpp_(float x) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, x), CTRL, 0xF, 0xF, false));
}
__device__ __forceinline__ float add_xor1(float x) { return x + dpp_<0xB1>(x); }    // quad_perm [1,0,3,2]
__device__ __forceinline__ float add_xor2(float x) { return x + dpp_<0x4E>(x); }    // quad_perm [2,3,0,1]
__device__ __forceinline__ float add_xor8(float x) { return x + dpp_<0x128>(x); }   // row_ror:8
// lane i <- lane 7 - i of its group of 8; after the quad sums this is the other quad's sum
__device__ __forceinline__ float add_halfmirror(float x) { return x + dpp_<0x141>(x); }
// v_permlane16_swap(x, x) hands each lane, in one of the two results, its own value and in the other the value
// of lane xor 16; their sum is the pair sum (likewise permlane32 for lane xor 32)
__device__ __forceinline__ float add_xor16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float add_xor32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
// sums over aligned lane groups of 8, 16, 32
__device__ __forceinline__ float sum8_dpp(float x) { return add_halfmirror(add_xor2(add_xor1(x))); }
__device__ __forceinline__ float sum16_dpp(float x) { return add_xor8(sum8_dpp(x)); }
__device__ __forceinline__ float sum32_dpp(float x) { return add_xor16(sum16_dpp(x)); }
// sum over the 8 lanes sharing lane & 7 (lane xor 8, 16, 32)
__device__ __forceinline__ float sum_stride8_dpp(float x) { return add_xor32(add_xor16(add_xor8(x))); }

// whole-wave sum and max. Every stage combines the same pairs of partial results as the xor butterfly
// 1, 2, 4, 8, 16, 32 (the half mirror pairs each quad with the other quad of its 8), so the result is
// bitwise that of the butterfly, on every lane.
__device__ __forceinline__ float wave_sum(float x) { return add_xor32(sum32_dpp(x)); }

typedef __attribute__((ext_vector_type(4))) float f32x4_n;

// ---- Per-head RMSNorm(1 + w) and partial rotate-half RoPE of one 256-wide bf16 head row per wave (square_rows +
// norm_rope, src/hs_guard/engine/fused_kernels.py:237-284). Lane l holds dims 4 l .. 4 l + 3 (x, 8 bytes) and their
// fp32 weights w4; cs / sn hold the rot / 2 rotary pairs, bf16-rounded. y = bf16(x * rsqrt(mean(x^2) + eps) * w);
// for d < rot: out = bf16(y cos) + bf16(rot_half(y) sin) (one fp32 add), else out = y. PM: the lane distance of
// a dim's rotate-half partner (rot / 8) when it is 8 (a DPP row rotate), 0 for any rot (a shuffle). Shared by
// hsg_norm_rope and the decode that applies it on the fly, so both give the same bits. ----
__device__ __forceinline__ void rope_pair(int64_t pos, float inv_freq, float& c, float& s) {
  const float f = (float)pos * inv_freq;
  c = rbf(cosf(f));
  s = rbf(sinf(f));
}

template <int PM>
__device__ __forceinline__ uint2 norm_rope_head256(uint2 xw, f32x4_n w4, float eps, const float* cs, const float* sn,
                                                  int rot, int lane) {
  const int half = rot / 2;
  const int d0 = 4 * lane;
  float x[4];
  unpack2(xw.x, x[0], x[1]);
  unpack2(xw.y, x[2], x[3]);
  const float ss = wave_sum(x[0] * x[0] + x[1] * x[1] + x[2] * x[2] + x[3] * x[3]);
  // 256 dims: ss / 256 is exactly ss * 2^-8
  const float r = rsqrtf(ss * (1.0f / 256.0f) + eps);
  float y[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) y[e] = rbf((x[e] * r) * w4[e]);
  float yp[4];
  if constexpr (PM == 8) {
#pragma unroll
    for (int e = 0; e < 4; ++e) yp[e] = dpp_<0x128>(y[e]);   // row_ror:8 is lane xor 8 within a 16-lane row
  } else {
#pragma unroll
    for (int e = 0; e < 4; ++e) yp[e] = __shfl_xor(y[e], half / 4, 64);
  }
  float o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) {
    const int d = d0 + e;
    if (d < rot) {
      const int fi = d < half ? d : d - half;
      const float rh = d < half ? -yp[e] : yp[e];
      o[e] = __fadd_rn(rbf(y[e] * cs[fi]), rbf(rh * sn[fi]));
    } else {
      o[e] = y[e];
    }
  }
  uint2 w;
  w.x = pack_bf16x2(o[0], o[1]);
  w.y = pack_bf16x2(o[2], o[3]);
  return w;
}

// ---- RMSNorm of one 1024-wide bf16 row per wave (add_square + rms_finish, src/hs_guard/engine/fused_kernels.py:
// 30-72). Lane l holds elements 8 l .. 8 l + 7 of the row in x[0] and 512 + 8 l .. + 7 in x[1] (16-byte pieces) and
// the matching fp32 weights w1 in w[0..3]. ADD: x = bf16(x + mix) first (one fp32 add; x is updated in place).
// Then out = bf16((x * rsqrt(mean(x^2) + eps)) * w1). Shared by hsg_add_rmsnorm and the skinny products that apply
// the norm while staging their operand, so both give the same bits. ----
__device__ __forceinline__ void unpack8(const u32x4& w, float* x) {
#pragma unroll
  for (int i = 0; i < 4; ++i) unpack2(w[i], x[2 * i], x[2 * i + 1]);
}

template <bool ADD>
__device__ __forceinline__ void rmsnorm_row1024(u32x4 (&x)[2], const u32x4 (&mix)[2], const f32x4_n (&w)[4],
                                                float eps, u32x4 (&out)[2]) {
  float h[16];
  unpack8(x[0], h);
  unpack8(x[1], h + 8);
  if constexpr (ADD) {
    float m[16];
    unpack8(mix[0], m);
    unpack8(mix[1], m + 8);
#pragma unroll
    for (int i = 0; i < 16; ++i) h[i] = rbf(__fadd_rn(h[i], m[i]));
    // h is bf16-exact: its bf16 bits are the upper half of the fp32 word
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      u32x4 o;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        o[i] = (__float_as_uint(h[8 * j + 2 * i]) >> 16) | (__float_as_uint(h[8 * j + 2 * i + 1]) & 0xffff0000u);
      x[j] = o;
    }
  }
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) ss += h[i] * h[i];
  ss = wave_sum(ss);
  const float r = rsqrtf(ss / 1024.0f + eps);
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    u32x4 o;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const f32x4_n wq = w[2 * j + (i >> 1)];
      o[i] = pack_bf16x2((h[8 * j + 2 * i] * r) * wq[(2 * i) & 3], (h[8 * j + 2 * i + 1] * r) * wq[(2 * i + 1) & 3]);
    }
    out[j] = o;
  }
}

__device__ __forceinline__ float max_pair16(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_pair32(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
// threadIdx.x through an empty asm: a code block called from several sites computes its own addresses from
// it at each (otherwise the compiler shares them between the sites and keeps them live across the loops in
// between, which costs registers).
__device__ __forceinline__ int tid_per_site() {
  int t = threadIdx.x;
  asm volatile("" : "+v"(t));
  return t;
}

// A loaded value through an empty asm: the load then runs where it stands. Without it the compiler sinks a load
// whose value only one side of a select uses into a branch, with its own wait, at every such select.
__device__ __forceinline__ float loaded_here(float x) {
  asm volatile("" : "+v"(x));
  return x;
}

__device__ __forceinline__ float wave_max(float x) {
  x = fmaxf(x, dpp_<0xB1>(x));
  x = fmaxf(x, dpp_<0x4E>(x));
  x = fmaxf(x, dpp_<0x141>(x));
  x = fmaxf(x, dpp_<0x128>(x));
  return max_pair32(max_pair16(x));
}

// workgroup barrier that orders LDS only (outstanding global loads stay in flight across it)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

inline bool aligned(const void* p, int bytes) { return (reinterpret_cast<uintptr_t>(p) % bytes) == 0; }

inline int launch_status() {
  hipError_t e = hipGetLastError();
  return e == hipSuccess ? HSG_OK : (int)e;
}

}  // namespace hsg
