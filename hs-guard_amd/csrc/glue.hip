// Per-token glue of the streaming step for gfx950: embedding + RMSNorm, residual add + RMSNorm,
// causal conv + SiLU with the per-slot conv-history update, per-head RMSNorm + partial RoPE, SiLU-mul,
// the two risk heads, and the ring_pos bookkeeping. Rounding points follow the reference's fused kernels
// (cited per kernel); every RMSNorm computes its variance in-kernel instead of a separate mean launch.
#include <math.h>

#include "hsg_common.h"

namespace hsg {
namespace {

// ---------------------------------------------------------------------------------------------------
// RMSNorm over a 1024-wide row, one wave per token. Lane l holds elements 8 l .. 8 l + 7 and 512 + 8 l .. +7, so
// each 16-byte load or store instruction of the wave covers 1 KB of the row; every load of the token (row, mix,
// weights) is issued before the first use, so a token costs one memory round trip.
// add_square + rms_finish (src/hs_guard/engine/fused_kernels.py:30-72): h = bf16(res + mix) (plain fp32
// add), out = bf16((h * rsqrt(mean(h^2) + eps)) * w1), w1 = 1 + weight in fp32.
// Embedding variant (slot_engine_v8.py:38,42-43): h = embedding row of the token id.
// ---------------------------------------------------------------------------------------------------
constexpr int HID = 1024;
typedef __attribute__((ext_vector_type(4))) float f32x4_;

template <bool EMBED, bool ADD>
__global__ __launch_bounds__(256) void rmsnorm_kernel(uint16_t* hidden, const uint16_t* mix, const int64_t* ids,
                                                      const uint16_t* emb, const float* w1, float eps,
                                                      uint16_t* normed, int tokens, int64_t vocab) {
  const int lane = threadIdx.x & 63;
  const int tok = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (tok >= tokens) return;
  const int64_t row = (int64_t)tok * HID;
  const uint16_t* src = hidden + row;
  if constexpr (EMBED) {
    int64_t id = ids[tok];
    if (id < 0 || id >= vocab) id = 0;  // out-of-vocab ids are rejected on the host; never read OOB
    src = emb + id * HID;
  }
  u32x4 hw[2], mw[2], o[2];
  f32x4_n wv[4];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int d = 8 * lane + 512 * j;
    hw[j] = *reinterpret_cast<const u32x4*>(src + d);
    mw[j] = ADD ? *reinterpret_cast<const u32x4*>(mix + row + d) : u32x4{0u, 0u, 0u, 0u};
    wv[2 * j] = *reinterpret_cast<const f32x4_n*>(w1 + d);
    wv[2 * j + 1] = *reinterpret_cast<const f32x4_n*>(w1 + d + 4);
  }
  rmsnorm_row1024<ADD>(hw, mw, wv, eps, o);
  if constexpr (EMBED || ADD) {
#pragma unroll
    for (int j = 0; j < 2; ++j) *reinterpret_cast<u32x4*>(hidden + row + 8 * lane + 512 * j) = hw[j];
  }
#pragma unroll
  for (int j = 0; j < 2; ++j) *reinterpret_cast<u32x4*>(normed + row + 8 * lane + 512 * j) = o[j];
}

// ---------------------------------------------------------------------------------------------------
// Causal depthwise conv (KS = 4) + SiLU with the conv-history pool update.
// _conv_silu_kernel (src/hs_guard/engine/fused_kernels.py:94-136): acc = sum_k w[c,k] * ext[t+k] in fp32,
// out = bf16(silu(bf16(acc))); when len > 0, pool[slot, i] = ext[len + i] for i < KS-1, where
// ext = [pool rows ; new tokens]. One thread per channel; the 3-row window slides in registers.
// ---------------------------------------------------------------------------------------------------
constexpr int KS = 4;

__global__ __launch_bounds__(256) void conv_silu_kernel(const uint16_t* qkv, int64_t qkv_stride, uint16_t* pool,
                                                        int64_t pool_rows, const uint16_t* weight,
                                                        const int64_t* slots, const int64_t* lens,
                                                        const int64_t* offsets, int L, int C, uint16_t* out,
                                                        int64_t out_stride) {
  const int n = blockIdx.y;
  const int c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= C) return;
  const int64_t slot = slots[n];
  int64_t len = lens[n];
  const bool padded = offsets == nullptr;
  const bool slot_ok = slot >= 0 && slot < pool_rows;
  if (!slot_ok || len < 0) len = 0;
  if (padded && len > L) len = L;
  const int steps = padded ? L : (int)len;
  if (!padded && len == 0) return;
  const int64_t tok0 = padded ? (int64_t)n * L : offsets[n];
  float w[KS];
  for (int k = 0; k < KS; ++k) w[k] = bf2f(weight[c * KS + k]);
  uint16_t e[KS - 1], keep[KS - 1];
  for (int i = 0; i < KS - 1; ++i) {
    e[i] = slot_ok ? pool[(slot * (KS - 1) + i) * (int64_t)C + c] : (uint16_t)0;
    keep[i] = e[i];
  }
  auto step = [&](int t, uint16_t x) {
    float acc = 0.f;
    acc = fmaf(w[0], bf2f(e[0]), acc);
    acc = fmaf(w[1], bf2f(e[1]), acc);
    acc = fmaf(w[2], bf2f(e[2]), acc);
    acc = fmaf(w[3], bf2f(x), acc);
    out[(tok0 + t) * out_stride + c] = f2bf(siluf_(rbf(acc)));
    e[0] = e[1];
    e[1] = e[2];
    e[2] = x;
    if (t == len - 1) {  // window after the last real token = ext[len .. len+2]
      keep[0] = e[0];
      keep[1] = e[1];
      keep[2] = e[2];
    }
  };
  // Whole batches of TB tokens load together (one memory round trip per batch instead of per token); the
  // remainder, which is all of a single-token row, goes one load at a time.
  constexpr int TB = 8;
  int t = 0;
  for (; t + TB <= steps; t += TB) {
    uint16_t xs[TB];
#pragma unroll
    for (int i = 0; i < TB; ++i) xs[i] = qkv[(tok0 + t + i) * qkv_stride + c];
#pragma unroll
    for (int i = 0; i < TB; ++i) step(t + i, xs[i]);
  }
  for (; t < steps; ++t) step(t, qkv[(tok0 + t) * qkv_stride + c]);
  if (len > 0) {
    for (int i = 0; i < KS - 1; ++i) pool[(slot * (KS - 1) + i) * (int64_t)C + c] = keep[i];
  }
}

// ---------------------------------------------------------------------------------------------------
// Gated RMSNorm of the GDN output, one wave per (token, head) of width 128 (2 values per lane).
// gated_finish (src/hs_guard/engine/fused_kernels.py:215-233), as the slot step's fused epilogue computes it:
// r = rsqrt(mean(o^2) + eps) over the head, out = bf16(bf16(w * bf16(o * r)) * silu(z)), o already bf16.
// ---------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gated_rmsnorm_kernel(const uint16_t* x, int64_t x_stride, const uint16_t* z,
                                                            int64_t z_stride, const uint16_t* w, float eps,
                                                            uint16_t* out, int64_t out_stride, int tokens,
                                                            int heads) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= tokens * heads) return;
  const int t = item / heads;
  const int c = (item - t * heads) * 128 + 2 * lane;
  float x0, x1, z0, z1, w0, w1;
  unpack2(*reinterpret_cast<const uint32_t*>(x + t * x_stride + c), x0, x1);
  unpack2(*reinterpret_cast<const uint32_t*>(z + t * z_stride + c), z0, z1);
  unpack2(*reinterpret_cast<const uint32_t*>(w + 2 * lane), w0, w1);
  const float ss = wave_sum(x0 * x0 + x1 * x1);
  const float r = rsqrtf(ss * (1.0f / 128) + eps);
  const float y0 = rbf(w0 * rbf(x0 * r)) * siluf_(z0);
  const float y1 = rbf(w1 * rbf(x1 * r)) * siluf_(z1);
  *reinterpret_cast<uint32_t*>(out + t * out_stride + c) = (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
}

// ---------------------------------------------------------------------------------------------------
// Per-head RMSNorm(1+w) + partial rotate-half RoPE for q and k in one launch, one workgroup per token.
// square_rows + norm_rope (src/hs_guard/engine/fused_kernels.py:237-284) with the rotary cos/sin of the
// Qwen3.5 rotary embedding computed in-kernel: freq = pos * inv_freq[i] (fp32), cos/sin rounded to bf16.
// y = bf16(x * rsqrt(mean(x^2)+eps) * w1); for d < rot: out = bf16(bf16(y*cos) + bf16(rot_half(y)*sin)).
// One workgroup per token; wave w handles heads w, w + 4, ... of q followed by k, 4 dims per lane. The rotary
// inputs are loaded first and every head row of the wave right after, all before the token's rot/2 cos/sin pairs
// are computed into LDS (every head of the token shares them), so one memory round trip covers the token.
// ---------------------------------------------------------------------------------------------------
struct RopeTensor {
  const uint16_t* src; int64_t src_row, src_head; int heads;
  const float* w1;
  uint16_t* out; int64_t out_row, out_head;
};

constexpr int ROPE_HEADS_PER_WAVE = 8;   // heads of q and k together per token: at most 4 x 8 = 32

// PM: the lane distance of a dim's rotate-half partner (rot / 8), 0 when only known at run time
template <int PM>
__global__ __launch_bounds__(256) void norm_rope_kernel(RopeTensor a, RopeTensor b, const int64_t* pos,
                                                        const float* inv_freq, int rot, float eps_a, float eps_b,
                                                        int tokens, int D) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int tok = blockIdx.x;
  const int half = rot / 2;
  __shared__ float cs_[128], sn_[128];   // rot <= D = 256
  const int heads_total = a.heads + b.heads;
  const int d0 = lane * 4;   // D / 64 = 4 dims per lane
  // loads retire in order, so the cos/sin wait only for the rotary inputs; rows past the last head reload the
  // last one and are not stored. Every load is unconditional (a tensor without heads reads the other's weights,
  // unused): a load under a branch made the compiler wait for all outstanding memory operations before each
  // head, the previous head's store included, one round trip per head.
  const int64_t tpos = pos[tok];
  const float ifreq = inv_freq[threadIdx.x & (half - 1)];
  const f32x4_n wa = *reinterpret_cast<const f32x4_n*>((a.heads ? a.w1 : b.w1) + d0);
  const f32x4_n wb = *reinterpret_cast<const f32x4_n*>((b.heads ? b.w1 : a.w1) + d0);
  __builtin_amdgcn_sched_barrier(0);   // keep these loads ahead of the rows'
  uint2 xw[ROPE_HEADS_PER_WAVE];
#pragma unroll
  for (int i = 0; i < ROPE_HEADS_PER_WAVE; ++i) {
    const int head = min(wave + 4 * i, heads_total - 1);
    const bool is_a = head < a.heads;
    const int hh = is_a ? head : head - a.heads;
    const uint16_t* src = is_a ? a.src + tok * a.src_row + hh * a.src_head : b.src + tok * b.src_row + hh * b.src_head;
    xw[i] = *reinterpret_cast<const uint2*>(src + d0);
  }
  if (threadIdx.x < half) rope_pair(tpos, ifreq, cs_[threadIdx.x], sn_[threadIdx.x]);
  lds_barrier();
#pragma unroll
  for (int i = 0; i < ROPE_HEADS_PER_WAVE; ++i) {
    const int head = wave + 4 * i;
    if (head < heads_total) {
      const bool is_a = head < a.heads;
      const int hh = is_a ? head : head - a.heads;
      const uint2 o = norm_rope_head256<PM>(xw[i], is_a ? wa : wb, is_a ? eps_a : eps_b, cs_, sn_, rot, lane);
      uint16_t* dst = is_a ? a.out + tok * a.out_row + hh * a.out_head : b.out + tok * b.out_row + hh * b.out_head;
      *reinterpret_cast<uint2*>(dst + d0) = o;
    }
  }
}

// ---------------------------------------------------------------------------------------------------
// SiLU-mul (src/hs_guard/engine/fused_kernels.py:76-90): out = bf16(bf16(silu(gate)) * up); gate and up
// are the two halves of the fused gate|up projection row.
// ---------------------------------------------------------------------------------------------------
__device__ __forceinline__ float lane_bf(const u32x4& v, int j) {   // bf16 element j of 8 packed in 16 bytes
  const uint32_t w = v[j >> 1];
  return __uint_as_float((j & 1) ? (w & 0xffff0000u) : (w << 16));
}

__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* gu, int64_t gu_stride, int width,
                                                       uint16_t* out) {
  // grid: x = 2,048-element column blocks of the row, y = token (no division of a flat index by the width)
  const int c = (blockIdx.x * 256 + threadIdx.x) * 8;
  if (c >= width) return;
  const int64_t tok = blockIdx.y;
  const u32x4 g = *reinterpret_cast<const u32x4*>(gu + tok * gu_stride + c);
  const u32x4 u = *reinterpret_cast<const u32x4*>(gu + tok * gu_stride + width + c);
  u32x4 y;
#pragma unroll
  for (int j = 0; j < 8; j += 2) {
    const float y0 = rbf(siluf_(lane_bf(g, j))) * lane_bf(u, j);
    const float y1 = rbf(siluf_(lane_bf(g, j + 1))) * lane_bf(u, j + 1);
    y[j >> 1] = (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
  }
  *reinterpret_cast<u32x4*>(out + tok * width + c) = y;
}

// ---------------------------------------------------------------------------------------------------
// Risk heads (src/hs_guard/runtime.py:61-74, src/hs_guard/engine/slot_engine_v7.py:58-61,
// slot_engine_v8.py:56): given y = bf16(Linear_1024->512(x) + b1) for each role (columns
// [role*512, role*512+512) of the fused projection), LayerNorm(512) in fp32, SiLU, round to bf16, Linear
// 512->3 with bf16 output, softmax in fp32. One wave per (token, role).
// ---------------------------------------------------------------------------------------------------
// One wave per (role, token). F32 = false: the streaming readout under autocast (slot_engine_v7.py:58-61): y is
// the bf16 output of the first Linear, LayerNorm in fp32 with fp32 parameters, SiLU rounded to bf16 (the input
// of the bf16 Linear), bf16 weights, bf16 logits. F32 = true: the complete-message readout (runtime.py:70-73),
// every operand and intermediate in fp32 and nothing rounded to bf16.
template <bool F32>
__global__ __launch_bounds__(256) void risk_head_kernel(const void* y_, int64_t y_stride, const float* ln_w,
                                                        const float* ln_b, const void* w2_, const void* b2_,
                                                        float eps, int roles, int width, float* probs, int tokens) {
  const int lane = threadIdx.x & 63;
  const int item = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (item >= tokens * roles) return;
  const int role = item / tokens;
  const int tok = item - role * tokens;
  constexpr int PL = 8;  // values per lane (width 512)
  const int d0 = lane * PL;
  float v[PL];
  if constexpr (F32) {
    const float* y = static_cast<const float*>(y_) + tok * y_stride + role * width + d0;
    for (int i = 0; i < PL; ++i) v[i] = y[i];
  } else {
    load8_bf16(static_cast<const uint16_t*>(y_) + tok * y_stride + role * width + d0, v);
  }
  float s = 0.f;
  for (int i = 0; i < PL; ++i) s += v[i];
  const float mean = wave_sum(s) / (float)width;
  float s2 = 0.f;
  for (int i = 0; i < PL; ++i) s2 += (v[i] - mean) * (v[i] - mean);
  const float rstd = rsqrtf(wave_sum(s2) / (float)width + eps);
  float a[PL];
  for (int i = 0; i < PL; ++i) {
    const float t = siluf_((v[i] - mean) * rstd * ln_w[role * width + d0 + i] + ln_b[role * width + d0 + i]);
    a[i] = F32 ? t : rbf(t);
  }
  float logit[3];
  for (int j = 0; j < 3; ++j) {
    float w[PL];
    if constexpr (F32) {
      const float* wp = static_cast<const float*>(w2_) + ((int64_t)role * 3 + j) * width + d0;
      for (int i = 0; i < PL; ++i) w[i] = wp[i];
    } else {
      load8_bf16(static_cast<const uint16_t*>(w2_) + ((int64_t)role * 3 + j) * width + d0, w);
    }
    float acc = 0.f;
    for (int i = 0; i < PL; ++i) acc += a[i] * w[i];
    if constexpr (F32) logit[j] = wave_sum(acc) + static_cast<const float*>(b2_)[role * 3 + j];
    else logit[j] = rbf(wave_sum(acc) + bf2f(static_cast<const uint16_t*>(b2_)[role * 3 + j]));
  }
  if (lane == 0) {
    const float m = fmaxf(logit[0], fmaxf(logit[1], logit[2]));
    const float e0 = expf(logit[0] - m), e1 = expf(logit[1] - m), e2 = expf(logit[2] - m);
    const float z = e0 + e1 + e2;
    float* dst = probs + ((int64_t)role * tokens + tok) * 3;
    dst[0] = e0 / z;
    dst[1] = e1 / z;
    dst[2] = e2 / z;
  }
}

// ---------------------------------------------------------------------------------------------------
// ring_pos[slot, (start + j) % W] = start + j for the valid steps of every row
// (src/hs_guard/engine/slot_engine_v8.py:41,57; column W stays -1).
// ---------------------------------------------------------------------------------------------------
__global__ void ring_pos_kernel(int64_t* ring_pos, int64_t ring_rows, const int64_t* slots, const int64_t* starts,
                                const int64_t* lens, int W, int lb_max) {
  const int n = blockIdx.x;
  const int64_t slot = slots[n];
  int64_t len = lens[n];
  if (slot < 0 || slot >= ring_rows || len <= 0) return;
  if (len > lb_max) len = lb_max;
  const int64_t start = starts[n];
  for (int j = threadIdx.x; j < len; j += blockDim.x) {
    const int64_t p = start + j;
    ring_pos[slot * (W + 1) + p % W] = p;
  }
}

}  // namespace
}  // namespace hsg

using namespace hsg;

extern "C" int hsg_embed_rmsnorm(const int64_t* ids, const void* emb, int64_t vocab, const float* w1, float eps,
                                 void* hidden, void* normed, int32_t tokens, int32_t width, void* stream) {
  if (tokens < 0 || width != 1024 || vocab <= 0) return tokens < 0 || vocab <= 0 ? HSG_ERR_ARG : HSG_ERR_SHAPE;
  if (tokens == 0) return HSG_OK;
  if (!ids || !emb || !w1 || !hidden || !normed) return HSG_ERR_ARG;
  if (!aligned(emb, 16) || !aligned(hidden, 16) || !aligned(normed, 16) || !aligned(w1, 16)) return HSG_ERR_ALIGN;
  hipLaunchKernelGGL((rmsnorm_kernel<true, false>), dim3((tokens + 3) / 4), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<uint16_t*>(hidden), nullptr, ids,
                     static_cast<const uint16_t*>(emb), w1, eps, static_cast<uint16_t*>(normed), tokens, vocab);
  return launch_status();
}

extern "C" int hsg_add_rmsnorm(void* hidden, const void* mix, const float* w1, float eps, void* normed,
                               int32_t tokens, int32_t width, void* stream) {
  if (tokens < 0) return HSG_ERR_ARG;
  if (width != 1024) return HSG_ERR_SHAPE;
  if (tokens == 0) return HSG_OK;
  if (!hidden || !w1 || !normed) return HSG_ERR_ARG;
  if (!aligned(hidden, 16) || (mix && !aligned(mix, 16)) || !aligned(normed, 16) || !aligned(w1, 16))
    return HSG_ERR_ALIGN;
  const dim3 grid((tokens + 3) / 4);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (mix)
    hipLaunchKernelGGL((rmsnorm_kernel<false, true>), grid, dim3(256), 0, s, static_cast<uint16_t*>(hidden),
                       static_cast<const uint16_t*>(mix), nullptr, nullptr, w1, eps, static_cast<uint16_t*>(normed),
                       tokens, (int64_t)0);
  else
    hipLaunchKernelGGL((rmsnorm_kernel<false, false>), grid, dim3(256), 0, s, static_cast<uint16_t*>(hidden),
                       nullptr, nullptr, nullptr, w1, eps, static_cast<uint16_t*>(normed), tokens, (int64_t)0);
  return launch_status();
}

extern "C" int hsg_conv_silu_update(const void* qkv, int64_t qkv_stride, void* pool, int64_t pool_rows,
                                    const void* weight, int32_t kernel_size, const int64_t* slots, const int64_t* lens,
                                    const int64_t* offsets, int32_t n_rows, int32_t L, int32_t channels, void* out,
                                    int64_t out_stride, void* stream) {
  if (n_rows < 0 || channels <= 0 || pool_rows <= 0 || L < 0) return HSG_ERR_ARG;
  if (kernel_size != KS) return HSG_ERR_SHAPE;
  if (n_rows == 0) return HSG_OK;
  if (!qkv || !pool || !weight || !slots || !lens || !out || (!offsets && L <= 0)) return HSG_ERR_ARG;
  const dim3 grid((channels + 255) / 256, n_rows);
  hipLaunchKernelGGL(conv_silu_kernel, grid, dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                     static_cast<const uint16_t*>(qkv), qkv_stride, static_cast<uint16_t*>(pool), pool_rows,
                     static_cast<const uint16_t*>(weight), slots, lens, offsets, L, channels,
                     static_cast<uint16_t*>(out), out_stride);
  return launch_status();
}

extern "C" int hsg_gated_rmsnorm(const void* x, int64_t x_stride, const void* z, int64_t z_stride, const void* w,
                                 float eps, void* out, int64_t out_stride, int32_t tokens, int32_t heads,
                                 int32_t width, void* stream) {
  if (tokens < 0 || heads < 0) return HSG_ERR_ARG;
  if (width != 128) return HSG_ERR_SHAPE;
  if (tokens == 0 || heads == 0) return HSG_OK;
  if (!x || !z || !w || !out) return HSG_ERR_ARG;
  if (x_stride % 2 || z_stride % 2 || out_stride % 2 || !aligned(x, 4) || !aligned(z, 4) || !aligned(w, 4) ||
      !aligned(out, 4))
    return HSG_ERR_ALIGN;
  const int64_t items = (int64_t)tokens * heads;
  hipLaunchKernelGGL(gated_rmsnorm_kernel, dim3((unsigned)((items + 3) / 4)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(x), x_stride,
                     static_cast<const uint16_t*>(z), z_stride, static_cast<const uint16_t*>(w), eps,
                     static_cast<uint16_t*>(out), out_stride, tokens, heads);
  return launch_status();
}

extern "C" int hsg_norm_rope(const void* q_src, int64_t q_row, int64_t q_head, int32_t q_heads, const float* q_w1,
                             float q_eps, void* q_out, int64_t q_out_row, int64_t q_out_head, const void* k_src,
                             int64_t k_row, int64_t k_head, int32_t k_heads, const float* k_w1, float k_eps,
                             void* k_out, int64_t k_out_row, int64_t k_out_head, const int64_t* pos,
                             const float* inv_freq, int32_t rot, int32_t tokens, int32_t head_dim, void* stream) {
  if (tokens < 0 || q_heads < 0 || k_heads < 0) return HSG_ERR_ARG;
  if (head_dim != 256 || rot <= 0 || rot > head_dim || rot % 8 != 0 || ((rot / 8) & (rot / 8 - 1)) != 0)
    return HSG_ERR_SHAPE;
  if (q_heads + k_heads > 32) return HSG_ERR_SHAPE;
  if (tokens == 0 || q_heads + k_heads == 0) return HSG_OK;
  if (!pos || !inv_freq || (q_heads && (!q_src || !q_w1 || !q_out)) || (k_heads && (!k_src || !k_w1 || !k_out)))
    return HSG_ERR_ARG;
  const int64_t strides[] = {q_row, q_head, q_out_row, q_out_head, k_row, k_head, k_out_row, k_out_head};
  for (int64_t s : strides)
    if (s % 4) return HSG_ERR_ALIGN;
  if ((q_heads && !aligned(q_w1, 16)) || (k_heads && !aligned(k_w1, 16))) return HSG_ERR_ALIGN;
  RopeTensor a{static_cast<const uint16_t*>(q_src), q_row, q_head, q_heads, q_w1, static_cast<uint16_t*>(q_out),
               q_out_row, q_out_head};
  RopeTensor b{static_cast<const uint16_t*>(k_src), k_row, k_head, k_heads, k_w1, static_cast<uint16_t*>(k_out),
               k_out_row, k_out_head};
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid((unsigned)tokens);
  if (rot == 64)
    hipLaunchKernelGGL(norm_rope_kernel<8>, grid, dim3(256), 0, st, a, b, pos, inv_freq, rot, q_eps, k_eps, tokens,
                       head_dim);
  else
    hipLaunchKernelGGL(norm_rope_kernel<0>, grid, dim3(256), 0, st, a, b, pos, inv_freq, rot, q_eps, k_eps, tokens,
                       head_dim);
  return launch_status();
}

extern "C" int hsg_silu_mul(const void* gate_up, int64_t row_stride, int32_t width, void* out, int32_t tokens,
                            void* stream) {
  if (tokens < 0 || width <= 0) return HSG_ERR_ARG;
  if (width % 8 || row_stride % 8) return HSG_ERR_ALIGN;
  if (tokens == 0) return HSG_OK;
  if (!gate_up || !out) return HSG_ERR_ARG;
  if (!aligned(gate_up, 16) || !aligned(out, 16)) return HSG_ERR_ALIGN;
  // at most 65,535 tokens per launch (the grid's y limit)
  for (int32_t t0 = 0; t0 < tokens; t0 += 65535)
    hipLaunchKernelGGL(silu_mul_kernel, dim3((unsigned)((width / 8 + 255) / 256), (unsigned)min(tokens - t0, 65535)),
                       dim3(256), 0, reinterpret_cast<hipStream_t>(stream),
                       static_cast<const uint16_t*>(gate_up) + (int64_t)t0 * row_stride, row_stride, width,
                       static_cast<uint16_t*>(out) + (int64_t)t0 * width);
  return launch_status();
}

extern "C" int hsg_risk_head(const void* y, int64_t y_stride, const float* ln_w, const float* ln_b, const void* w2,
                             const void* b2, float eps, int32_t roles, int32_t width, float* probs, int32_t tokens,
                             void* stream) {
  if (tokens < 0 || roles <= 0) return HSG_ERR_ARG;
  if (width != 512) return HSG_ERR_SHAPE;
  if (tokens == 0) return HSG_OK;
  if (!y || !ln_w || !ln_b || !w2 || !b2 || !probs) return HSG_ERR_ARG;
  if (y_stride % 8 || !aligned(y, 16) || !aligned(ln_w, 4) || !aligned(ln_b, 4) || !aligned(w2, 16))
    return HSG_ERR_ALIGN;
  const int items = tokens * roles;
  hipLaunchKernelGGL(risk_head_kernel<false>, dim3((items + 3) / 4), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), y, y_stride, ln_w, ln_b, w2, b2, eps, roles, width, probs,
                     tokens);
  return launch_status();
}

extern "C" int hsg_risk_head_f32(const float* y, int64_t y_stride, const float* ln_w, const float* ln_b,
                                 const float* w2, const float* b2, float eps, int32_t roles, int32_t width,
                                 float* probs, int32_t tokens, void* stream) {
  if (tokens < 0 || roles <= 0) return HSG_ERR_ARG;
  if (width != 512) return HSG_ERR_SHAPE;
  if (tokens == 0) return HSG_OK;
  if (!y || !ln_w || !ln_b || !w2 || !b2 || !probs) return HSG_ERR_ARG;
  if (!aligned(y, 4) || !aligned(ln_w, 4) || !aligned(ln_b, 4) || !aligned(w2, 4)) return HSG_ERR_ALIGN;
  const int items = tokens * roles;
  hipLaunchKernelGGL(risk_head_kernel<true>, dim3((items + 3) / 4), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), y, y_stride, ln_w, ln_b, w2, b2, eps, roles, width, probs,
                     tokens);
  return launch_status();
}

extern "C" int hsg_ring_pos_update(int64_t* ring_pos, int64_t ring_rows, int32_t window, const int64_t* slots,
                                   const int64_t* starts, const int64_t* lens, int32_t n_rows, int32_t lb_max,
                                   void* stream) {
  if (n_rows < 0 || window <= 0 || ring_rows <= 0 || lb_max <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  if (!ring_pos || !slots || !starts || !lens) return HSG_ERR_ARG;
  hipLaunchKernelGGL(ring_pos_kernel, dim3(n_rows), dim3(64), 0, reinterpret_cast<hipStream_t>(stream), ring_pos,
                     ring_rows, slots, starts, lens, window, lb_max);
  return launch_status();
}
