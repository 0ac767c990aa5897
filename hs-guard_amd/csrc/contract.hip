// Unfused glue kernels with the reference engine's own kernel contracts, for callers that compose the step the way
// the reference's SlotStreamEngineV8 does (src/hs_guard/engine/slot_engine_v8.py:30-89): the variance of every
// RMSNorm arrives as an input (the caller's sq.mean(-1)), the rotary cos/sin arrive precomputed, SiLU-mul takes
// separate gate and up tensors, and q/k leave RMSNorm + RoPE in the grouped [N, Hkv, G*Lb, D] layout of the ring
// kernel. The streaming engine of this library runs the fused forms instead (glue.hip); both follow the same
// rounding points of src/hs_guard/engine/fused_kernels.py.
//
// Every kernel here is element-wise once the per-row variance is given, so each thread owns VEC consecutive
// elements of one row (VEC = 4: 8-byte bf16 loads and 16-byte fp32 stores, used when the row width and every
// pointer allow it; VEC = 1 otherwise), and rows of any width and count work.
#include <math.h>

#include "hsg_common.h"

namespace hsg {
namespace {

constexpr int CT_THREADS = 256;

template <int VEC>
__device__ __forceinline__ void load_bf(const uint16_t* p, float* x) {
  if constexpr (VEC == 4) {
    load4_bf16(p, x);
  } else {
    x[0] = bf2f(p[0]);
  }
}

template <int VEC>
__device__ __forceinline__ void store_bf(uint16_t* p, const float* x) {
  if constexpr (VEC == 4) {
    store4_bf16(p, x);
  } else {
    p[0] = f2bf(x[0]);
  }
}

template <int VEC>
__device__ __forceinline__ void store_f32(float* p, const float* x) {
  if constexpr (VEC == 4) {
    *reinterpret_cast<float4*>(p) = make_float4(x[0], x[1], x[2], x[3]);
  } else {
    p[0] = x[0];
  }
}

template <int VEC>
__device__ __forceinline__ int64_t first_element(int64_t n) {
  const int64_t i = ((int64_t)blockIdx.x * CT_THREADS + threadIdx.x) * VEC;
  return i < n ? i : -1;
}

// add_square (src/hs_guard/engine/fused_kernels.py:30-52): h = bf16(res + mix) with a plain fp32 add (no
// contraction), stored when mix is given; sq = h^2 in fp32 (of res when mix is NULL).
template <int VEC>
__global__ __launch_bounds__(CT_THREADS) void add_square_kernel(const uint16_t* res, const uint16_t* mix,
                                                                uint16_t* out, float* sq, int64_t n) {
  const int64_t i = first_element<VEC>(n);
  if (i < 0) return;
  float h[VEC];
  load_bf<VEC>(res + i, h);
  if (mix) {
    float m[VEC];
    load_bf<VEC>(mix + i, m);
#pragma unroll
    for (int e = 0; e < VEC; ++e) h[e] = rbf(__fadd_rn(h[e], m[e]));
    store_bf<VEC>(out + i, h);
  }
#pragma unroll
  for (int e = 0; e < VEC; ++e) h[e] = h[e] * h[e];
  store_f32<VEC>(sq + i, h);
}

// rms_finish (fused_kernels.py:56-72): out = bf16((x * rsqrt(var[row] + eps)) * w1[col]).
template <int VEC>
__global__ __launch_bounds__(CT_THREADS) void rms_finish_kernel(const uint16_t* x, const float* var, const float* w1,
                                                                float eps, uint16_t* out, int64_t n, int width) {
  const int64_t i = first_element<VEC>(n);
  if (i < 0) return;
  const int64_t row = i / width;
  const int col = (int)(i - row * width);
  float h[VEC];
  load_bf<VEC>(x + i, h);
  const float r = rsqrtf(var[row] + eps);
#pragma unroll
  for (int e = 0; e < VEC; ++e) h[e] = (h[e] * r) * w1[col + e];
  store_bf<VEC>(out + i, h);
}

// silu_mul (fused_kernels.py:76-90): out = bf16(bf16(silu(gate)) * up) over two tensors of n elements.
template <int VEC>
__global__ __launch_bounds__(CT_THREADS) void silu_mul_pair_kernel(const uint16_t* gate, const uint16_t* up,
                                                                   uint16_t* out, int64_t n) {
  const int64_t i = first_element<VEC>(n);
  if (i < 0) return;
  float g[VEC], u[VEC];
  load_bf<VEC>(gate + i, g);
  load_bf<VEC>(up + i, u);
#pragma unroll
  for (int e = 0; e < VEC; ++e) g[e] = rbf(siluf_(g[e])) * u[e];
  store_bf<VEC>(out + i, g);
}

// gated_finish (fused_kernels.py:215-233): out = bf16(bf16(w[col] * bf16(x * rsqrt(var[row] + eps))) * silu(z)).
template <int VEC>
__global__ __launch_bounds__(CT_THREADS) void gated_finish_kernel(const uint16_t* x, const float* var,
                                                                  const uint16_t* w, const uint16_t* z, float eps,
                                                                  uint16_t* out, int64_t n, int width) {
  const int64_t i = first_element<VEC>(n);
  if (i < 0) return;
  const int64_t row = i / width;
  const int col = (int)(i - row * width);
  float h[VEC], g[VEC], wv[VEC];
  load_bf<VEC>(x + i, h);
  load_bf<VEC>(z + i, g);
  load_bf<VEC>(w + col, wv);
  const float r = rsqrtf(var[row] + eps);
#pragma unroll
  for (int e = 0; e < VEC; ++e) h[e] = rbf(wv[e] * rbf(h[e] * r)) * siluf_(g[e]);
  store_bf<VEC>(out + i, h);
}

// square_rows (fused_kernels.py:237-249): sq[r, c] = x^2 of head r % heads of token r / heads, read from the
// strided projection rows; sq is [tokens * heads, dim] fp32.
template <int VEC>
__global__ __launch_bounds__(CT_THREADS) void square_rows_kernel(const uint16_t* src, float* sq, int heads,
                                                                 int64_t row_stride, int64_t head_stride, int dim,
                                                                 int64_t n) {
  const int64_t i = first_element<VEC>(n);
  if (i < 0) return;
  const int64_t r = i / dim;
  const int c = (int)(i - r * dim);
  const int64_t token = r / heads;
  const int j = (int)(r - token * heads);
  float x[VEC];
  load_bf<VEC>(src + token * row_stride + j * head_stride + c, x);
#pragma unroll
  for (int e = 0; e < VEC; ++e) x[e] = x[e] * x[e];
  store_f32<VEC>(sq + i, x);
}

// norm_rope (fused_kernels.py:252-284): per-head RMSNorm(1 + w) given var, then rotate-half RoPE on the first rot
// dims with the given bf16 cos/sin [tokens, rot]:
//   x = bf16((src[d] * rsqrt(var + eps)) * w1[d]), xp the same at d's partner (d +- rot/2),
//   out[d] = bf16(bf16(x * cos) + bf16(+-xp * sin)) for d < rot, bf16(x) beyond,
// written at out + n*out_n + (j / groups)*out_h + ((j % groups)*lb + l)*out_row + d for head j of token n*lb + l.
// One thread per element; the partner is a second (cached) load of the same row.
__global__ __launch_bounds__(CT_THREADS) void norm_rope_grouped_kernel(
    const uint16_t* src, const float* var, const float* w1, const uint16_t* cosv, const uint16_t* sinv, int rot,
    float eps, int heads, int lb, int groups, int64_t row_stride, int64_t head_stride, int dim, uint16_t* out,
    int64_t out_n, int64_t out_h, int64_t out_row, int64_t n) {
  const int64_t i = first_element<1>(n);
  if (i < 0) return;
  const int64_t r = i / dim;
  const int d = (int)(i - r * dim);
  const int64_t token = r / heads;
  const int j = (int)(r - token * heads);
  const int64_t nn = token / lb;
  const int l = (int)(token - nn * lb);
  const int half = rot / 2;
  const int partner = d < half ? d + half : (d < rot ? d - half : d);
  const float rr = rsqrtf(var[r] + eps);
  const uint16_t* base = src + token * row_stride + j * head_stride;
  const float x = rbf((bf2f(base[d]) * rr) * w1[d]);
  float y = x;
  if (d < rot) {
    const float xp = rbf((bf2f(base[partner]) * rr) * w1[partner]);
    const float c = bf2f(cosv[token * rot + d]);
    const float s = bf2f(sinv[token * rot + d]);
    const float rh = d < half ? -xp : xp;
    y = __fadd_rn(rbf(x * c), rbf(rh * s));
  }
  out[nn * out_n + (j / groups) * out_h + ((int64_t)(j % groups) * lb + l) * out_row + d] = f2bf(y);
}

unsigned blocks_for(int64_t n, int vec) {
  return (unsigned)((n / vec + CT_THREADS - 1) / CT_THREADS);
}

// VEC = 4 needs rows of a multiple of 4 elements and 8-byte aligned bf16 / 16-byte aligned fp32 pointers
bool vec4_ok(int64_t width, std::initializer_list<const void*> bf, std::initializer_list<const void*> f32) {
  if (width % 4) return false;
  for (const void* p : bf)
    if (p && !aligned(p, 8)) return false;
  for (const void* p : f32)
    if (p && !aligned(p, 16)) return false;
  return true;
}

}  // namespace
}  // namespace hsg

using namespace hsg;

extern "C" int hsg_add_square(const void* residual, const void* mixed, void* out, float* sq, int64_t rows,
                              int32_t width, void* stream) {
  if (rows < 0 || width <= 0) return HSG_ERR_ARG;
  if (rows == 0) return HSG_OK;
  if (!residual || !sq || (mixed && !out)) return HSG_ERR_ARG;
  const int64_t n = rows * width;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto* r = static_cast<const uint16_t*>(residual);
  const auto* m = static_cast<const uint16_t*>(mixed);
  auto* o = static_cast<uint16_t*>(out);
  if (vec4_ok(width, {residual, mixed, out}, {sq}))
    hipLaunchKernelGGL(add_square_kernel<4>, dim3(blocks_for(n, 4)), dim3(CT_THREADS), 0, s, r, m, o, sq, n);
  else
    hipLaunchKernelGGL(add_square_kernel<1>, dim3(blocks_for(n, 1)), dim3(CT_THREADS), 0, s, r, m, o, sq, n);
  return launch_status();
}

extern "C" int hsg_rms_finish(const void* x, const float* var, const float* w1, float eps, void* out, int64_t rows,
                              int32_t width, void* stream) {
  if (rows < 0 || width <= 0) return HSG_ERR_ARG;
  if (rows == 0) return HSG_OK;
  if (!x || !var || !w1 || !out) return HSG_ERR_ARG;
  const int64_t n = rows * width;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto* xi = static_cast<const uint16_t*>(x);
  auto* o = static_cast<uint16_t*>(out);
  if (vec4_ok(width, {x, out}, {}))
    hipLaunchKernelGGL(rms_finish_kernel<4>, dim3(blocks_for(n, 4)), dim3(CT_THREADS), 0, s, xi, var, w1, eps, o, n,
                       width);
  else
    hipLaunchKernelGGL(rms_finish_kernel<1>, dim3(blocks_for(n, 1)), dim3(CT_THREADS), 0, s, xi, var, w1, eps, o, n,
                       width);
  return launch_status();
}

extern "C" int hsg_silu_mul_pair(const void* gate, const void* up, void* out, int64_t n, void* stream) {
  if (n < 0) return HSG_ERR_ARG;
  if (n == 0) return HSG_OK;
  if (!gate || !up || !out) return HSG_ERR_ARG;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto* g = static_cast<const uint16_t*>(gate);
  const auto* u = static_cast<const uint16_t*>(up);
  auto* o = static_cast<uint16_t*>(out);
  if (vec4_ok(n, {gate, up, out}, {}))
    hipLaunchKernelGGL(silu_mul_pair_kernel<4>, dim3(blocks_for(n, 4)), dim3(CT_THREADS), 0, s, g, u, o, n);
  else
    hipLaunchKernelGGL(silu_mul_pair_kernel<1>, dim3(blocks_for(n, 1)), dim3(CT_THREADS), 0, s, g, u, o, n);
  return launch_status();
}

extern "C" int hsg_gated_finish(const void* x, const float* var, const void* weight, const void* z, float eps,
                                void* out, int64_t rows, int32_t width, void* stream) {
  if (rows < 0 || width <= 0) return HSG_ERR_ARG;
  if (rows == 0) return HSG_OK;
  if (!x || !var || !weight || !z || !out) return HSG_ERR_ARG;
  const int64_t n = rows * width;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto* xi = static_cast<const uint16_t*>(x);
  const auto* w = static_cast<const uint16_t*>(weight);
  const auto* zi = static_cast<const uint16_t*>(z);
  auto* o = static_cast<uint16_t*>(out);
  if (vec4_ok(width, {x, weight, z, out}, {}))
    hipLaunchKernelGGL(gated_finish_kernel<4>, dim3(blocks_for(n, 4)), dim3(CT_THREADS), 0, s, xi, var, w, zi, eps, o,
                       n, width);
  else
    hipLaunchKernelGGL(gated_finish_kernel<1>, dim3(blocks_for(n, 1)), dim3(CT_THREADS), 0, s, xi, var, w, zi, eps, o,
                       n, width);
  return launch_status();
}

extern "C" int hsg_square_rows(const void* src, float* sq, int64_t tokens, int32_t heads, int64_t row_stride,
                               int64_t head_stride, int32_t dim, void* stream) {
  if (tokens < 0 || heads <= 0 || dim <= 0 || row_stride < 0 || head_stride < 0) return HSG_ERR_ARG;
  if (tokens == 0) return HSG_OK;
  if (!src || !sq) return HSG_ERR_ARG;
  const int64_t n = tokens * heads * dim;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const auto* x = static_cast<const uint16_t*>(src);
  if (vec4_ok(dim, {src}, {sq}) && row_stride % 4 == 0 && head_stride % 4 == 0)
    hipLaunchKernelGGL(square_rows_kernel<4>, dim3(blocks_for(n, 4)), dim3(CT_THREADS), 0, s, x, sq, heads,
                       row_stride, head_stride, dim, n);
  else
    hipLaunchKernelGGL(square_rows_kernel<1>, dim3(blocks_for(n, 1)), dim3(CT_THREADS), 0, s, x, sq, heads,
                       row_stride, head_stride, dim, n);
  return launch_status();
}

extern "C" int hsg_norm_rope_grouped(const void* src, const float* var, const float* w1, const void* cos,
                                     const void* sin, int32_t rot, float eps, int32_t n_rows, int32_t lb,
                                     int32_t heads, int32_t groups, int64_t row_stride, int64_t head_stride,
                                     int32_t dim, void* out, int64_t out_n, int64_t out_h, int64_t out_row,
                                     void* stream) {
  if (n_rows < 0 || lb <= 0 || heads <= 0 || groups <= 0 || dim <= 0) return HSG_ERR_ARG;
  if (heads % groups || rot <= 0 || rot % 2 || rot > dim) return HSG_ERR_SHAPE;
  if (n_rows == 0) return HSG_OK;
  if (!src || !var || !w1 || !cos || !sin || !out) return HSG_ERR_ARG;
  const int64_t n = (int64_t)n_rows * lb * heads * dim;
  hipLaunchKernelGGL(norm_rope_grouped_kernel, dim3(blocks_for(n, 1)), dim3(CT_THREADS), 0,
                     reinterpret_cast<hipStream_t>(stream), static_cast<const uint16_t*>(src), var, w1,
                     static_cast<const uint16_t*>(cos), static_cast<const uint16_t*>(sin), rot, eps, heads, lb,
                     groups, row_stride, head_stride, dim, static_cast<uint16_t*>(out), out_n, out_h, out_row, n);
  return launch_status();
}
