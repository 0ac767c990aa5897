// Window-W GQA ring attention for decode steps (one query position per row) on gfx950.
//
// Contract and numerics: those of hsg_ring_attention (src/hs_guard/engine/fused_kernels.py:288-376 and the
// torch reference src/hs_guard/engine/ring_attention_kernel.py:7-26) for rows with lens[n] == 1: keys in
// blocks of 32 (ring columns in order, then the step's own key), a running max m_b over the blocks,
// probabilities p = exp(s - m_b) rounded to bf16 in the P.V product and summed unrounded, output / sum
// rounded to bf16, times bf16(sigmoid(gate)). The running max of block b is the prefix maximum of the block
// maxima, and the reference's rescaling chain multiplies block b's P.V and sum by exp(m_b - m_final), so the
// blocks can be processed by different waves or workgroups without changing where any bf16 rounding happens.
//
// Up to 8 query heads per kv head: decode_fused_kernel, one launch, one workgroup per (row, kv head) with every
// score and partial sum in LDS (no workspace traffic). More heads per kv head: three split-K launches over a
// workspace:
//   A (scores):  (row, kv head, split) -> s = scale * q.k for the split's ring blocks (masked -inf) and each
//                block's maximum per query head, into the workspace; the last split adds the step's own key.
//   B (values):  (row, kv head, split) -> prefix maxima from all block maxima, then for each of its blocks
//                exp(m_b - m_final) * sum_k bf16(exp(s_k - m_b)) v_k and the matching unrounded sum.
//   C (combine): (row, kv head) -> sum over splits, divide, gate, store; then the in-place ring write of the
//                step's key and value (every read of this ring finished in B).
// Blocks with no visible key are skipped (no K or V traffic) on both paths. The split is over the 512 ring
// columns: 4 splits of 4 blocks, one block per wave.
#include <math.h>

#include <mutex>

#include "hsg_common.h"

namespace hsg {
namespace {

constexpr int D = 256;
constexpr int KB = 32;             // keys per softmax block
constexpr int NS = 4;              // splits of the ring columns
constexpr int W_MAX = 512;
constexpr int G_MAX = 16;          // query heads per kv head

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2;
typedef __attribute__((ext_vector_type(4))) float f32x4;

// exp of a softmax argument or rescale exponent on the hardware exp2 (v_exp_f32): exp(x) = 2^(x log2 e), as the
// reference kernel's tl.exp (src/hs_guard/engine/fused_kernels.py:318-319,335-336).
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

// value of lane l (l uniform over the wave): v_readlane, no LDS round trip
__device__ __forceinline__ float readlane_f(float x, int l) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, x), l));
}

struct DecParams {
  const uint16_t* q; int64_t q_sn, q_sl, q_sh, q_sg;
  uint16_t* ring_k; uint16_t* ring_v; int64_t ring_rows; int W;
  const uint16_t* new_k; int64_t nk_sn, nk_sl, nk_sh;
  const uint16_t* new_v; int64_t nv_sn, nv_sl, nv_sh;
  const uint16_t* gate; int64_t g_sn, g_sl, g_sh, g_sg, g_off;
  const int64_t* ring_pos; const int64_t* slots; const int64_t* starts; const int64_t* lens;
  const int64_t* offsets;
  int hkv, G;
  float scale;
  int write_ring;
  uint16_t* out; int64_t o_sn, o_sl, o_sh, o_sg;
  float* ws;
  int64_t unit;     // floats of workspace per (row, kv head)
  int sc_stride;    // floats per query head in the score area (W + KB)
  // hsg_ring_decode_rope: raw q / k rows, their norm weights and the rotary inputs; the scores kernel normalises
  // and rotates them itself and writes the new keys to k_out (read back as new_k by the combine kernel)
  const uint16_t* q_raw; int64_t qr_sl, qr_sh;
  const uint16_t* k_raw; int64_t kr_sl, kr_sh;
  const float* q_w1; const float* k_w1; float q_eps, k_eps;
  const int64_t* pos; const float* inv_freq; int rot;
  uint16_t* k_out;
};

// Workspace of one (row, kv head): scores [G][W + KB] | block maxima [G][KB] | partial sums [NS][G][D] |
// partial normalisers [NS][G] (padded).
__host__ __device__ inline int64_t unit_floats(int G, int W) {
  const int64_t f = (int64_t)G * (W + KB) + (int64_t)G * KB + (int64_t)NS * G * D + (int64_t)NS * G_MAX;
  return (f + 63) / 64 * 64;
}

struct RowInfo {
  bool live;          // lens == 1 and a valid slot
  int64_t slot, start, tok;
};

__device__ __forceinline__ RowInfo row_info(const DecParams& p, int n) {
  RowInfo r;
  r.slot = p.slots[n];
  r.start = p.starts[n];
  r.live = p.lens[n] == 1 && r.slot >= 0 && r.slot < p.ring_rows;
  r.tok = p.offsets ? p.offsets[n] : n;
  return r;
}

__device__ __forceinline__ int64_t row_base(const DecParams& p, int64_t sn, int64_t sl, int n, int64_t tok) {
  return p.offsets ? tok * sl : (int64_t)n * sn;
}

// ---------------------------------------------------------------------------------------------------------
// ROPE (hsg_ring_decode_rope, packed layout): the kv head's G queries and the step's own key arrive raw; the
// workgroup first gives each the per-head RMSNorm(1 + w) and rotate-half RoPE of hsg_norm_rope (the same
// norm_rope_head256, one head row per wave, so the bits are those of the separate launch) into LDS, and the last
// split's workgroup writes the new key to k_out for the combine kernel's ring write.
template <bool ROPE>
__global__ __launch_bounds__(256) void decode_scores_kernel(const DecParams p) {
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m16 = lane & 15, g4 = lane >> 4;
  const int s = blockIdx.x % NS;
  const int u = blockIdx.x / NS;
  const int n = u / p.hkv, h = u - n * p.hkv;
  const RowInfo ri = row_info(p, n);
  if (!ri.live) return;
  const int W = p.W, G = p.G, RB = W / KB;
  const int bps = (RB + NS - 1) / NS;
  const int b = s * bps + wave;
  float* sc = p.ws + u * p.unit;
  float* bm = sc + (int64_t)G * p.sc_stride;
  const int64_t qpos = ri.start;
  const uint16_t* qrow = p.q + row_base(p, p.q_sn, p.q_sl, n, ri.tok) + h * p.q_sh;
  __shared__ __align__(16) uint16_t qr_s[ROPE ? G_MAX * D : 8];   // the group's queries, normalised and rotated
  __shared__ __align__(16) uint16_t kr_s[ROPE ? D : 8];           // the step's own key, likewise
  __shared__ float cs_s[ROPE ? D / 2 : 1], sn_s[ROPE ? D / 2 : 1];
  if constexpr (ROPE) {
    // items 0 .. G - 1: query heads h G + g; item G: the own key. Wave w takes items w, w + 4, ...; every load is
    // issued before the rotary pairs are computed.
    constexpr int IT = (G_MAX + 1 + 3) / 4;
    uint2 xw[IT];
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int item = min(wave + 4 * i, G);
      const uint16_t* src = item < G ? p.q_raw + ri.tok * p.qr_sl + (h * G + item) * p.qr_sh
                                     : p.k_raw + ri.tok * p.kr_sl + h * p.kr_sh;
      xw[i] = *reinterpret_cast<const uint2*>(src + 4 * lane);
    }
    const f32x4_n wq = *reinterpret_cast<const f32x4_n*>(p.q_w1 + 4 * lane);
    const f32x4_n wk = *reinterpret_cast<const f32x4_n*>(p.k_w1 + 4 * lane);
    if (threadIdx.x < p.rot / 2)
      rope_pair(p.pos[ri.tok], p.inv_freq[threadIdx.x], cs_s[threadIdx.x], sn_s[threadIdx.x]);
    lds_barrier();
#pragma unroll
    for (int i = 0; i < IT; ++i) {
      const int item = wave + 4 * i;
      if (item <= G) {   // wave-uniform
        const bool is_q = item < G;
        const uint2 o = norm_rope_head256<8>(xw[i], is_q ? wq : wk, is_q ? p.q_eps : p.k_eps, cs_s, sn_s, p.rot, lane);
        if (is_q) {
          *reinterpret_cast<uint2*>(&qr_s[item * D + 4 * lane]) = o;
        } else {
          *reinterpret_cast<uint2*>(&kr_s[4 * lane]) = o;
          if (s == NS - 1)
            *reinterpret_cast<uint2*>(p.k_out + row_base(p, p.nk_sn, p.nk_sl, n, ri.tok) + h * p.nk_sh + 4 * lane) = o;
        }
      }
    }
    lds_barrier();
  }

  if (wave < bps && b < RB) {
    // Two memory round trips: the block's positions (and the queries), then its keys only if one of them
    // is visible (a partly filled ring costs no key traffic for its empty blocks).
    const int64_t* rpos = p.ring_pos + ri.slot * (int64_t)(W + 1) + b * KB;
    int64_t kp8[2][4];
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) kp8[t][r] = rpos[16 * t + 4 * g4 + r];
    // B operand: query head m16 (zero for m16 >= G), dims 32 ks + 8 g4 ..
    bf16x8 qb[D / 32];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (m16 < G)
        w = ROPE ? *reinterpret_cast<const uint4*>(&qr_s[m16 * D + 32 * ks + 8 * g4])
                 : *reinterpret_cast<const uint4*>(qrow + m16 * p.q_sg + 32 * ks + 8 * g4);
      qb[ks] = __builtin_bit_cast(bf16x8, w);
    }
    bool vis = false;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) vis |= kp8[t][r] >= 0 && kp8[t][r] <= qpos && kp8[t][r] > qpos - W;
    if (__ballot(vis) == 0) {
      if (lane < G) bm[lane * KB + b] = -INFINITY;
    } else {
      const uint16_t* kbase = p.ring_k + ((ri.slot * p.hkv + h) * (int64_t)(W + 1) + b * KB) * D;
      uint4 ka[2][D / 32];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks)
          ka[t][ks] = *reinterpret_cast<const uint4*>(kbase + (16 * t + m16) * D + 32 * ks + 8 * g4);
      float bmax = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks)
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[t][ks]), qb[ks], acc, 0, 0, 0);
        // lane (query m16, keys 16 t + 4 g4 + r)
        f32x4 sv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int64_t kp = kp8[t][r];
          const bool ok = kp >= 0 && kp <= qpos && kp > qpos - W;
          sv[r] = ok ? acc[r] * p.scale : -INFINITY;
          bmax = fmaxf(bmax, sv[r]);
        }
        if (m16 < G) *reinterpret_cast<f32x4*>(sc + m16 * p.sc_stride + b * KB + 16 * t + 4 * g4) = sv;
      }
      bmax = max_pair32(max_pair16(bmax));   // over g4 (lane xor 16, 32)
      if (g4 == 0 && m16 < G) bm[m16 * KB + b] = bmax;
    }
  }

  // the step's own key: block RB, one key, always visible to its own query
  if (s == NS - 1 && wave == 0) {
    const uint16_t* kn = ROPE ? kr_s : p.new_k + row_base(p, p.nk_sn, p.nk_sl, n, ri.tok) + h * p.nk_sh;
    float k4[4];
    load4_bf16(kn + 4 * lane, k4);
    for (int g = 0; g < G; ++g) {
      float q4[4];
      load4_bf16(ROPE ? qr_s + g * D + 4 * lane : qrow + g * p.q_sg + 4 * lane, q4);
      const float part = q4[0] * k4[0] + q4[1] * k4[1] + q4[2] * k4[2] + q4[3] * k4[3];
      const float v = wave_sum(part) * p.scale;
      if (lane == 0) {
        sc[g * p.sc_stride + W] = v;
        bm[g * KB + RB] = v;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
template <int GT>
__global__ __launch_bounds__(256) void decode_values_kernel(const DecParams p) {
  __shared__ __align__(16) float pb_s[4][GT][KB];
  __shared__ __align__(16) float red[4][GT * D / 4][4];
  __shared__ float lsum_s[4][GT];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int s = blockIdx.x % NS;
  const int u = blockIdx.x / NS;
  const int n = u / p.hkv, h = u - n * p.hkv;
  const RowInfo ri = row_info(p, n);
  if (!ri.live) return;
  const int W = p.W, G = p.G, RB = W / KB, NB = RB + 1;
  const int bps = (RB + NS - 1) / NS;
  const int b = s * bps + wave;
  float* sc = p.ws + u * p.unit;
  const float* bm = sc + (int64_t)G * p.sc_stride;
  float* pacc = const_cast<float*>(bm) + (int64_t)G * KB;
  float* pl = pacc + (int64_t)NS * G * D;

  // Two memory round trips: every block maximum of the lane's head (lanes g < G) and the block's scores
  // (lane: head g0 + lane / 16, keys 2 (lane % 16), +1) together, then the block's values (lane: dims
  // 8 (lane % 32) .., keys 2 j + lane / 32) only if one of its keys is visible.
  const bool ring_block = wave < bps && b < RB;
  const int dl = 8 * (lane & 31), kh = lane >> 5;
  float bmv[W_MAX / KB + 1];
#pragma unroll
  for (int j = 0; j <= W_MAX / KB; ++j) bmv[j] = (lane < G && j < NB) ? bm[lane * KB + j] : -INFINITY;
  constexpr int GR = (GT + 3) / 4;   // rounds of 4 heads for the probabilities
  float sv[GR][2];
#pragma unroll
  for (int gr = 0; gr < GR; ++gr) {
    const int g = 4 * gr + (lane >> 4);
    const int key = 2 * (lane & 15);
    sv[gr][0] = sv[gr][1] = -INFINITY;
    if (ring_block && g < G) {
      const float2 x = *reinterpret_cast<const float2*>(sc + g * p.sc_stride + b * KB + key);
      sv[gr][0] = x.x;
      sv[gr][1] = x.y;
    }
  }
  // lane g < G: running max through block b (m_b) and over all blocks (m_final)
  float mb = -INFINITY, mf = -INFINITY;
#pragma unroll
  for (int j = 0; j <= W_MAX / KB; ++j) {
    mf = fmaxf(mf, bmv[j]);
    if (j == b) mb = mf;
  }
  float acc[GT][8];
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[g][i] = 0.f;
  float lpart = 0.f;   // lane g < G: this wave's weighted normaliser for head g

  // a block without any visible key has no scores written (every head shares the step's visibility)
  const bool has_block = ring_block && readlane_f(bmv[b < NB ? b : 0], 0) != -INFINITY;
  if (has_block) {
    const float mb_l = mb;
    uint4 vr[KB / 2];
    const uint16_t* vbase = p.ring_v + ((ri.slot * p.hkv + h) * (int64_t)(W + 1) + b * KB) * D + dl;
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) vr[j] = *reinterpret_cast<const uint4*>(vbase + (2 * j + kh) * D);
#pragma unroll
    for (int gr = 0; gr < GR; ++gr) {
      const int g0 = 4 * gr;
      const int g = g0 + (lane >> 4);
      const int key = 2 * (lane & 15);
      const float m_g = __shfl(mb_l, g < G ? g : 0, 64);
      float p0 = 0.f, p1 = 0.f;
      if (g < G && m_g != -INFINITY) {
        p0 = sv[gr][0] == -INFINITY ? 0.f : exp_fast(sv[gr][0] - m_g);
        p1 = sv[gr][1] == -INFINITY ? 0.f : exp_fast(sv[gr][1] - m_g);
      }
      if (g < G) {
        pb_s[wave][g][key] = rbf(p0);
        pb_s[wave][g][key + 1] = rbf(p1);
      }
      float ps = p0 + p1;   // unrounded, as the reference's row sum
      ps = sum16_dpp(ps);
      // lane 16 j holds the sum for head g0 + j; move it to lane g0 + j
      const float got = __shfl(ps, 16 * ((lane - g0) & 3), 64);
      if (lane >= g0 && lane < g0 + 4 && lane < G) lpart = got;
    }
    // block weight exp(m_b - m_final) per head (lane g < G)
    float wgt = 0.f;
    if (lane < G && mb_l != -INFINITY) wgt = exp_fast(mb_l - mf);
    lpart *= wgt;
    __builtin_amdgcn_wave_barrier();
#pragma unroll
    for (int j = 0; j < KB / 2; ++j) {
      const int k = 2 * j + kh;
      float v[8];
      unpack2(vr[j].x, v[0], v[1]);
      unpack2(vr[j].y, v[2], v[3]);
      unpack2(vr[j].z, v[4], v[5]);
      unpack2(vr[j].w, v[6], v[7]);
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        if (g < G) {
          const float pk = pb_s[wave][g][k];
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] += pk * v[i];
        }
      }
    }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (g < G) {
        const float wg = readlane_f(wgt, g);
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[g][i] = add_xor32(acc[g][i]) * wg;  // both key halves (lane xor 32)
      }
    }
  }

  // the step's own key (block RB): last split, wave 0; its running max is m_final, weight 1
  if (s == NS - 1 && wave == 0) {
    const uint16_t* vn = p.new_v + row_base(p, p.nv_sn, p.nv_sl, n, ri.tok) + h * p.nv_sh + dl;
    float v[8];
    load4_bf16(vn, v);
    load4_bf16(vn + 4, v + 4);
    float pnew = 0.f;
    if (lane < G) pnew = exp_fast(sc[lane * p.sc_stride + W] - mf);
    lpart += pnew;
    if (kh == 0) {
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        if (g < G) {
          const float pk = rbf(readlane_f(pnew, g));
#pragma unroll
          for (int i = 0; i < 8; ++i) acc[g][i] += pk * v[i];
        }
      }
    }
  }

  // ---- reduce the four waves (lanes < 32 hold dims 8 lane .. 8 lane + 7) ----
  if (kh == 0) {
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (g < G) {
        float* dst = &red[wave][g * (D / 4) + 2 * lane][0];
        *reinterpret_cast<float4*>(dst) = make_float4(acc[g][0], acc[g][1], acc[g][2], acc[g][3]);
        *reinterpret_cast<float4*>(dst + 4) = make_float4(acc[g][4], acc[g][5], acc[g][6], acc[g][7]);
      }
    }
  }
  if (lane < G) lsum_s[wave][lane] = lpart;
  __syncthreads();
  for (int e = threadIdx.x; e < G * (D / 4); e += 256) {
    float4 t = make_float4(0.f, 0.f, 0.f, 0.f);
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float4 x = *reinterpret_cast<const float4*>(&red[w][e][0]);
      t.x += x.x; t.y += x.y; t.z += x.z; t.w += x.w;
    }
    *reinterpret_cast<float4*>(pacc + (int64_t)s * G * D + 4 * e) = t;
  }
  if (threadIdx.x < G) {
    pl[s * G_MAX + threadIdx.x] = lsum_s[0][threadIdx.x] + lsum_s[1][threadIdx.x] + lsum_s[2][threadIdx.x] +
                                  lsum_s[3][threadIdx.x];
  }
}

// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void decode_combine_kernel(const DecParams p) {
  const int u = blockIdx.x;
  const int n = u / p.hkv, h = u - n * p.hkv;
  const RowInfo ri = row_info(p, n);
  const int W = p.W, G = p.G;
  if (!ri.live) {
    // padded layout: a row without a live step (lens 0 or a rejected slot) owns an output row of zeros
    if (p.offsets == nullptr) {
      for (int e = threadIdx.x; e < G * (D / 4); e += 256) {
        const int g = e / (D / 4), d = 4 * (e - g * (D / 4));
        const float z[4] = {0.f, 0.f, 0.f, 0.f};
        store4_bf16(p.out + (int64_t)n * p.o_sn + h * p.o_sh + g * p.o_sg + d, z);
      }
    }
    return;
  }
  const float* sc = p.ws + u * p.unit;
  const float* pacc = sc + (int64_t)G * p.sc_stride + (int64_t)G * KB;
  const float* pl = pacc + (int64_t)NS * G * D;
  uint16_t* orow = p.out + row_base(p, p.o_sn, p.o_sl, n, ri.tok) + h * p.o_sh;
  const uint16_t* grow = p.gate ? p.gate + row_base(p, p.g_sn, p.g_sl, n, ri.tok) + h * p.g_sh + p.g_off : nullptr;
  for (int e = threadIdx.x; e < G * (D / 4); e += 256) {
    const int g = e / (D / 4), d = 4 * (e - g * (D / 4));
    float o[4] = {0.f, 0.f, 0.f, 0.f};
    float l = 0.f;
#pragma unroll
    for (int s = 0; s < NS; ++s) {
      const float4 x = *reinterpret_cast<const float4*>(pacc + (int64_t)s * G * D + g * D + d);
      o[0] += x.x; o[1] += x.y; o[2] += x.z; o[3] += x.w;
      l += pl[s * G_MAX + g];
    }
    float y[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) y[i] = l > 0.f ? rbf(o[i] / l) : 0.f;
    if (grow) {
      float gt[4];
      load4_bf16(grow + g * p.g_sg + d, gt);
#pragma unroll
      for (int i = 0; i < 4; ++i) y[i] = y[i] * rbf(1.0f / (1.0f + expf(-gt[i])));
    }
    store4_bf16(orow + g * p.o_sg + d, y);
  }
  if (p.write_ring) {
    const int64_t col = ri.start % W;
    const int64_t dst = ((ri.slot * p.hkv + h) * (int64_t)(W + 1) + col) * D;
    const uint16_t* kn = p.new_k + row_base(p, p.nk_sn, p.nk_sl, n, ri.tok) + h * p.nk_sh;
    const uint16_t* vn = p.new_v + row_base(p, p.nv_sn, p.nv_sl, n, ri.tok) + h * p.nv_sh;
    for (int e = threadIdx.x; e < 2 * (D / 4); e += 256) {
      const int which = e / (D / 4), d = 4 * (e - which * (D / 4));
      if (which == 0) *reinterpret_cast<uint2*>(p.ring_k + dst + d) = *reinterpret_cast<const uint2*>(kn + d);
      else *reinterpret_cast<uint2*>(p.ring_v + dst + d) = *reinterpret_cast<const uint2*>(vn + d);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Fused decode (groups <= 8): one workgroup of 4 waves per (row, kv head), wave w owning ring blocks w, w + 4,
// w + 8 and w + 12 (32 keys each), so every score, block maximum and partial sum stays in LDS and the whole step is
// one launch. The numerics are those of the three split-K kernels above (same block maxima, prefix maxima, bf16
// probabilities and block weights); only the fp32 summation order of the partial P.V sums differs (keys in order
// within a block, the wave's blocks in order, then a fixed tree over the waves). Memory: round trip 1 issues the
// blocks' positions, the queries (into LDS) and the step's own key and value; then each visible block's keys, one
// block at a time; the first block's values go out as soon as the scores are done and are in flight across the
// block-maximum barrier, each later block's after the previous block's P.V. Several of these workgroups share a
// CU, so one workgroup's loads cover another's barriers and arithmetic.
template <int GT>
__global__ __launch_bounds__(256) void decode_fused_kernel(const DecParams p) {
  constexpr int NWV = 4;                       // waves
  constexpr int BPW = W_MAX / KB / NWV;        // ring blocks per wave (4)
  constexpr int NBK = W_MAX / KB;              // ring blocks (16)
  constexpr int GR = (GT + 3) / 4;             // rounds of 4 heads for the probabilities
  __shared__ __align__(16) uint16_t q_s[GT * D];            // queries of the kv head's group, head-major
  __shared__ __align__(16) float sc_s[GT][W_MAX];           // scale q.k per ring column (-inf where masked)
  __shared__ float bm_s[GT][NBK + 1];                       // block maxima; column RB: the step's own key
  __shared__ float own_s[GT];                               // the step's own-key score
  __shared__ __align__(16) uint32_t pb_s[NBK][GT][KB / 2];  // bf16 probabilities, key pairs (2 j, 2 j + 1)
  __shared__ __align__(16) float red_s[NWV / 2][GT][D];     // reduction tree of the per-wave P.V partials
  __shared__ float lsum_s[NWV][GT];                         // per-wave weighted normalisers
  __shared__ uint2 vown_s[64];                              // the step's own value (lane: dims 4 lane .. +3)

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int m16 = lane & 15, g4 = lane >> 4;
  const int u = blockIdx.x;
  const int n = u / p.hkv, h = u - n * p.hkv;
  const RowInfo ri = row_info(p, n);
  const int W = p.W, G = p.G, RB = W / KB;
  if (!ri.live) {
    // padded layout: a row without a live step (lens 0 or a rejected slot) owns an output row of zeros
    if (p.offsets == nullptr) {
      for (int e = threadIdx.x; e < G * (D / 4); e += 64 * NWV) {
        const int g = e / (D / 4), d = 4 * (e - g * (D / 4));
        const float z[4] = {0.f, 0.f, 0.f, 0.f};
        store4_bf16(p.out + (int64_t)n * p.o_sn + h * p.o_sh + g * p.o_sg + d, z);
      }
    }
    return;
  }
  const int64_t qpos = ri.start;
  const uint16_t* qrow = p.q + row_base(p, p.q_sn, p.q_sl, n, ri.tok) + h * p.q_sh;
  const int64_t ring_at = (ri.slot * p.hkv + h) * (int64_t)(W + 1);

  // ---- round trip 1: queries into LDS, the blocks' positions, the step's own key and value. Every load here is
  // unconditional (addresses clamped in bounds, what a thread does not need discarded) and issued before the
  // first use: loads under branches were compiled as one wait per branch, five round trips instead of one. ----
  const int qc = threadIdx.x % (D / 8);
  const uint4 qw = *reinterpret_cast<const uint4*>(qrow + min((int)threadIdx.x / (D / 8), G - 1) * p.q_sg + 8 * qc);
  int64_t kp[BPW][2][4];
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int64_t* rpos = p.ring_pos + ri.slot * (int64_t)(W + 1) + min(wave + NWV * i, RB - 1) * KB;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) kp[i][t][r] = rpos[16 * t + 4 * g4 + r];
  }
  const uint2 kown = *reinterpret_cast<const uint2*>(p.new_k + row_base(p, p.nk_sn, p.nk_sl, n, ri.tok) +
                                                     h * p.nk_sh + 4 * lane);
  const uint2 vown = *reinterpret_cast<const uint2*>(p.new_v + row_base(p, p.nv_sn, p.nv_sl, n, ri.tok) +
                                                     h * p.nv_sh + 4 * lane);
  if (threadIdx.x < GT * D / 8) {
    const int g = threadIdx.x / (D / 8);
    *reinterpret_cast<uint4*>(&q_s[g * D + 8 * qc]) = g < G ? qw : make_uint4(0u, 0u, 0u, 0u);
  }
  uint32_t okbits = 0;   // bit 8 i + 4 t + r: key 16 t + 4 g4 + r of block i is visible
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const bool in_ring = wave + NWV * i < RB;
#pragma unroll
    for (int t = 0; t < 2; ++t)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t k = kp[i][t][r];
        okbits |= (uint32_t)(in_ring && k >= 0 && k <= qpos && k > qpos - W) << (8 * i + 4 * t + r);
      }
  }
  const bool own_wave = wave == NWV - 1;
  if (own_wave) vown_s[lane] = vown;   // parked in LDS until the end, where it is the last value added
  bool has[BPW];   // wave-uniform: block i has a visible key (false past the ring)
#pragma unroll
  for (int i = 0; i < BPW; ++i) has[i] = __ballot(((okbits >> (8 * i)) & 0xffu) != 0) != 0;
  lds_barrier();   // B0: queries in LDS

  // ---- scores, one block at a time (A: keys, lane keys 16 t + m16, dims 32 ks + 8 g4 ..; B: queries m16 < G
  // from LDS): lane (query m16, keys 16 t + 4 g4 + r) ----
  uint2 vr[KB];    // values of the block in P.V, lane: dims 4 lane .. +3 of key k
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int b = wave + NWV * i;
    if (has[i]) {
      const uint16_t* kbase = p.ring_k + (ring_at + b * KB) * D;
      uint4 ka[2][D / 32];
#pragma unroll
      for (int t = 0; t < 2; ++t)
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks)
          ka[t][ks] = ld_stream16(kbase + (16 * t + m16) * D + 32 * ks + 8 * g4);
      float bmax = -INFINITY;
#pragma unroll
      for (int t = 0; t < 2; ++t) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < D / 32; ++ks) {
          uint4 w = make_uint4(0u, 0u, 0u, 0u);
          if (m16 < GT) w = *reinterpret_cast<const uint4*>(&q_s[m16 * D + 32 * ks + 8 * g4]);
          acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, ka[t][ks]),
                                                        __builtin_bit_cast(bf16x8, w), acc, 0, 0, 0);
        }
        f32x4 sv;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          sv[r] = ((okbits >> (8 * i + 4 * t + r)) & 1u) ? acc[r] * p.scale : -INFINITY;
          bmax = fmaxf(bmax, sv[r]);
        }
        if (m16 < G) *reinterpret_cast<f32x4*>(&sc_s[m16][b * KB + 16 * t + 4 * g4]) = sv;
      }
      bmax = max_pair32(max_pair16(bmax));   // over g4 (lane xor 16, 32)
      if (g4 == 0 && m16 < G) bm_s[m16][b] = bmax;
    } else if (b < RB && lane < G) {
      bm_s[lane][b] = -INFINITY;
    }
  }
  if (has[0]) {
    // the first block's values go out now (the keys' registers are free) and arrive across the barriers
    const uint16_t* vbase = p.ring_v + (ring_at + wave * KB) * D + 4 * lane;
#pragma unroll
    for (int k = 0; k < KB; ++k) vr[k] = ld_stream8(vbase + k * D);
  }
  if (own_wave) {
    // the step's own key: block RB, one key, always visible to its own query
    float k4[4];
    unpack2(kown.x, k4[0], k4[1]);
    unpack2(kown.y, k4[2], k4[3]);
    for (int g = 0; g < G; ++g) {
      const uint2 qw = *reinterpret_cast<const uint2*>(&q_s[g * D + 4 * lane]);
      float q4[4];
      unpack2(qw.x, q4[0], q4[1]);
      unpack2(qw.y, q4[2], q4[3]);
      const float part = q4[0] * k4[0] + q4[1] * k4[1] + q4[2] * k4[2] + q4[3] * k4[3];
      const float v = wave_sum(part) * p.scale;
      if (lane == 0) {
        own_s[g] = v;
        bm_s[g][RB] = v;
      }
    }
  }
  lds_barrier();   // B1: every score and block maximum is in LDS

  // ---- lane g < G: running max through each of the wave's blocks (m_b) and over all blocks and the own key
  // (m_final); then each block's probabilities into LDS and its weight exp(m_b - m_final) ----
  float mb[BPW], mf = -INFINITY;
#pragma unroll
  for (int i = 0; i < BPW; ++i) mb[i] = -INFINITY;
  if (lane < G) {
    for (int j = 0; j <= RB; ++j) {
      mf = fmaxf(mf, bm_s[lane][j]);
#pragma unroll
      for (int i = 0; i < BPW; ++i)
        if (j == wave + NWV * i) mb[i] = mf;
    }
  }
  float lpart = 0.f;   // lane g < G: this wave's weighted normaliser for head g
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int b = wave + NWV * i;
    if (!has[i]) continue;
    const float wgt = (lane < G && mb[i] != -INFINITY) ? exp_fast(mb[i] - mf) : 0.f;
    float li = 0.f;
#pragma unroll
    for (int gr = 0; gr < GR; ++gr) {
      const int g0 = 4 * gr;
      const int g = g0 + (lane >> 4);
      const int key = 2 * (lane & 15);
      const float m_g = __shfl(mb[i], g < G ? g : 0, 64);
      float p0 = 0.f, p1 = 0.f;
      if (g < G && m_g != -INFINITY) {
        const float2 sv = *reinterpret_cast<const float2*>(&sc_s[g][b * KB + key]);
        p0 = sv.x == -INFINITY ? 0.f : exp_fast(sv.x - m_g);
        p1 = sv.y == -INFINITY ? 0.f : exp_fast(sv.y - m_g);
      }
      // bf16 probabilities as key pairs (rows g >= G hold zeros, so P.V runs over all GT rows without a
      // per-head test)
      pb_s[b][g][lane & 15] = pack_bf16x2(p0, p1);
      float ps = p0 + p1;   // unrounded, as the reference's row sum
      ps = sum16_dpp(ps);
      // lane 16 j holds the sum for head g0 + j; move it to lane g0 + j
      const float got = __shfl(ps, 16 * ((lane - g0) & 3), 64);
      if (lane >= g0 && lane < g0 + 4 && lane < G) li = got;
    }
    lpart += li * wgt;
  }
  lds_barrier();   // B2: the probabilities are in LDS (read back by every lane of the wave)

  // ---- P.V, lane: dims 4 lane .. +3. The wave's blocks are chained as in the reference's rescaling:
  // acc <- acc exp(m_prev - m_b) + P_b.V_b, then one final factor exp(m_last - m_final), so each block's sum is
  // weighted by exp(m_b - m_final). Two keys per v_dot2_f32_bf16: probabilities (p_2j, p_2j+1) against values
  // (v_2j[d], v_2j+1[d]), the value pairs assembled with byte permutes. ----
  float acc[GT][4];
#pragma unroll
  for (int g = 0; g < GT; ++g)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[g][e] = 0.f;
  float mprev = -INFINITY;   // lane g < G: running max of the last block added
#pragma unroll
  for (int i = 0; i < BPW; ++i) {
    const int b = wave + NWV * i;
    if (!has[i]) continue;
    if (i > 0) {
      const uint16_t* vbase = p.ring_v + (ring_at + b * KB) * D + 4 * lane;
#pragma unroll
      for (int k = 0; k < KB; ++k) vr[k] = ld_stream8(vbase + k * D);
    }
    const float alpha = (lane < G && mb[i] != -INFINITY) ? exp_fast(mprev - mb[i]) : 0.f;
    if (lane < G) mprev = mb[i];
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float a_g = readlane_f(alpha, g < G ? g : 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[g][e] *= a_g;
    }
#pragma unroll
    for (int j2 = 0; j2 < KB / 2; j2 += 2) {
      uint2 pp[GT];
#pragma unroll
      for (int g = 0; g < GT; ++g) pp[g] = *reinterpret_cast<const uint2*>(&pb_s[b][g][j2]);
#pragma unroll
      for (int jj = 0; jj < 2; ++jj) {
        const uint2 a = vr[2 * (j2 + jj)], c = vr[2 * (j2 + jj) + 1];
        const uint32_t vp[4] = {__builtin_amdgcn_perm(c.x, a.x, 0x05040100u), __builtin_amdgcn_perm(c.x, a.x, 0x07060302u),
                                __builtin_amdgcn_perm(c.y, a.y, 0x05040100u), __builtin_amdgcn_perm(c.y, a.y, 0x07060302u)};
#pragma unroll
        for (int g = 0; g < GT; ++g) {
          const uint32_t pg = jj == 0 ? pp[g].x : pp[g].y;
#pragma unroll
          for (int e = 0; e < 4; ++e)
            acc[g][e] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2, pg),
                                                        __builtin_bit_cast(bf16x2, vp[e]), acc[g][e], false);
        }
      }
    }
  }
  {
    const float wl = (lane < G && mprev != -INFINITY) ? exp_fast(mprev - mf) : 0.f;
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float w_g = readlane_f(wl, g < G ? g : 0);
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[g][e] *= w_g;
    }
  }
  if (own_wave) {
    // the own key's running max is m_final and its weight 1
    float pown = 0.f;
    if (lane < G) pown = exp_fast(own_s[lane] - mf);
    lpart += pown;
    const uint2 vo = vown_s[lane];
    float v[4];
    unpack2(vo.x, v[0], v[1]);
    unpack2(vo.y, v[2], v[3]);
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      const float pk = rbf(readlane_f(pown, g));   // 0 for g >= G
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[g][e] += pk * v[e];
    }
  }
  if (lane < G) lsum_s[wave][lane] = lpart;

  // ---- fixed reduction tree over the waves: wave w + half adds into wave w ----
#pragma unroll
  for (int half = NWV / 2; half >= 1; half >>= 1) {
    if (wave >= half && wave < 2 * half) {
#pragma unroll
      for (int g = 0; g < GT; ++g)
        *reinterpret_cast<f32x4*>(&red_s[wave - half][g][4 * lane]) =
            (f32x4){acc[g][0], acc[g][1], acc[g][2], acc[g][3]};
    }
    lds_barrier();
    if (wave < half) {
#pragma unroll
      for (int g = 0; g < GT; ++g) {
        const f32x4 x = *reinterpret_cast<const f32x4*>(&red_s[wave][g][4 * lane]);
#pragma unroll
        for (int e = 0; e < 4; ++e) acc[g][e] += x[e];
      }
    }
    lds_barrier();
  }

  // ---- wave 0: normalise, gate, store; wave 1: the in-place ring write (every read of this ring is done) ----
  if (wave == 0) {
    uint16_t* orow = p.out + row_base(p, p.o_sn, p.o_sl, n, ri.tok) + h * p.o_sh;
    const uint16_t* grow = p.gate ? p.gate + row_base(p, p.g_sn, p.g_sl, n, ri.tok) + h * p.g_sh + p.g_off
                                  : nullptr;
    // every head's gate piece is loaded before the first output store (out may alias gate as far as the compiler
    // knows, so a load after a store waits for it: one memory round trip per head otherwise)
    uint2 gw[GT];
    if (grow) {
#pragma unroll
      for (int g = 0; g < GT; ++g)
        gw[g] = *reinterpret_cast<const uint2*>(grow + min(g, G - 1) * p.g_sg + 4 * lane);
    }
#pragma unroll
    for (int g = 0; g < GT; ++g) {
      if (g < G) {
        float l = 0.f;
        for (int w = 0; w < NWV; ++w) l += lsum_s[w][g];
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = l > 0.f ? rbf(acc[g][e] / l) : 0.f;
        if (grow) {
          float gt[4];
          unpack2(gw[g].x, gt[0], gt[1]);
          unpack2(gw[g].y, gt[2], gt[3]);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = y[e] * rbf(1.0f / (1.0f + expf(-gt[e])));
        }
        store4_bf16(orow + g * p.o_sg + 4 * lane, y);
      }
    }
  } else if (wave == 1 && p.write_ring) {
    const int64_t dst = (ring_at + ri.start % W) * D + 4 * lane;
    const uint16_t* kn = p.new_k + row_base(p, p.nk_sn, p.nk_sl, n, ri.tok) + h * p.nk_sh + 4 * lane;
    const uint16_t* vn = p.new_v + row_base(p, p.nv_sn, p.nv_sl, n, ri.tok) + h * p.nv_sh + 4 * lane;
    *reinterpret_cast<uint2*>(p.ring_k + dst) = *reinterpret_cast<const uint2*>(kn);
    *reinterpret_cast<uint2*>(p.ring_v + dst) = *reinterpret_cast<const uint2*>(vn);
  }
}

}  // namespace
}  // namespace hsg

extern "C" size_t hsg_ring_decode_workspace_bytes(int32_t n_rows, int32_t hkv, int32_t groups, int32_t window) {
  if (n_rows <= 0 || hkv <= 0 || groups <= 0 || window <= 0) return 0;
  return (size_t)n_rows * hkv * (size_t)hsg::unit_floats(groups, window) * sizeof(float);
}

extern "C" int hsg_ring_decode(const void* q, int64_t q_sn, int64_t q_sl, int64_t q_sh, int64_t q_sg,
                               void* ring_k, void* ring_v, int64_t ring_rows, int32_t window,
                               const void* new_k, int64_t nk_sn, int64_t nk_sl, int64_t nk_sh,
                               const void* new_v, int64_t nv_sn, int64_t nv_sl, int64_t nv_sh,
                               const void* gate, int64_t g_sn, int64_t g_sl, int64_t g_sh, int64_t g_sg,
                               int64_t g_off, const int64_t* ring_pos, const int64_t* slots,
                               const int64_t* starts, const int64_t* lens, const int64_t* offsets,
                               int32_t n_rows, int32_t hkv, int32_t groups, int32_t head_dim, float scale,
                               int32_t write_ring, void* out, int64_t o_sn, int64_t o_sl, int64_t o_sh,
                               int64_t o_sg, void* workspace, size_t workspace_bytes, void* stream) {
  using namespace hsg;
  if (n_rows < 0 || hkv <= 0 || groups <= 0 || ring_rows <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  // the split-K path: always above 8 query heads per kv head; up to 8 for a few rows when the caller gives a workspace
  // (a row's ring then spreads over 4 workgroups). The fused kernel neither needs nor reads the workspace.
  const bool split = groups > 8 || (workspace && (int64_t)n_rows * hkv <= HSG_RING_DECODE_SPLIT_UNITS &&
                                    workspace_bytes >= hsg_ring_decode_workspace_bytes(n_rows, hkv, groups, window));
  if (!q || !ring_k || !ring_v || !new_k || !new_v || !ring_pos || !slots || !starts || !lens || !out ||
      (split && !workspace))
    return HSG_ERR_ARG;
  if (head_dim != D || window <= 0 || window > W_MAX || window % KB != 0 || groups > G_MAX) return HSG_ERR_SHAPE;
  if (split && workspace_bytes < hsg_ring_decode_workspace_bytes(n_rows, hkv, groups, window)) return HSG_ERR_SHAPE;
  const int64_t s16[] = {q_sn, q_sl, q_sh, q_sg};
  for (int64_t s : s16)
    if (s % 8) return HSG_ERR_ALIGN;
  const int64_t s4[] = {nk_sn, nk_sl, nk_sh, nv_sn, nv_sl, nv_sh, g_sn, g_sl, g_sh, g_sg, g_off, o_sn, o_sl, o_sh, o_sg};
  for (int64_t s : s4)
    if (s % 4) return HSG_ERR_ALIGN;
  if (!aligned(q, 16) || !aligned(ring_k, 16) || !aligned(ring_v, 16) || !aligned(new_k, 8) ||
      !aligned(new_v, 8) || !aligned(out, 8) || (gate && !aligned(gate, 8)) || (split && !aligned(workspace, 16)))
    return HSG_ERR_ALIGN;
  DecParams p{};
  p.q = static_cast<const uint16_t*>(q); p.q_sn = q_sn; p.q_sl = q_sl; p.q_sh = q_sh; p.q_sg = q_sg;
  p.ring_k = static_cast<uint16_t*>(ring_k); p.ring_v = static_cast<uint16_t*>(ring_v);
  p.ring_rows = ring_rows; p.W = window;
  p.new_k = static_cast<const uint16_t*>(new_k); p.nk_sn = nk_sn; p.nk_sl = nk_sl; p.nk_sh = nk_sh;
  p.new_v = static_cast<const uint16_t*>(new_v); p.nv_sn = nv_sn; p.nv_sl = nv_sl; p.nv_sh = nv_sh;
  p.gate = static_cast<const uint16_t*>(gate);
  p.g_sn = g_sn; p.g_sl = g_sl; p.g_sh = g_sh; p.g_sg = g_sg; p.g_off = g_off;
  p.ring_pos = ring_pos; p.slots = slots; p.starts = starts; p.lens = lens; p.offsets = offsets;
  p.hkv = hkv; p.G = groups; p.scale = scale; p.write_ring = write_ring;
  p.out = static_cast<uint16_t*>(out); p.o_sn = o_sn; p.o_sl = o_sl; p.o_sh = o_sh; p.o_sg = o_sg;
  p.ws = static_cast<float*>(workspace);
  p.unit = unit_floats(groups, window);
  p.sc_stride = window + KB;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned units = (unsigned)(n_rows * hkv);
  if (!split) {
    if (groups <= 4) hipLaunchKernelGGL(decode_fused_kernel<4>, dim3(units), dim3(256), 0, st, p);
    else hipLaunchKernelGGL(decode_fused_kernel<8>, dim3(units), dim3(256), 0, st, p);
    return launch_status();
  }
  hipLaunchKernelGGL(decode_scores_kernel<false>, dim3(units * NS), dim3(256), 0, st, p);
  if (groups <= 4) hipLaunchKernelGGL(decode_values_kernel<4>, dim3(units * NS), dim3(256), 0, st, p);
  else if (groups <= 8) hipLaunchKernelGGL(decode_values_kernel<8>, dim3(units * NS), dim3(256), 0, st, p);
  else hipLaunchKernelGGL(decode_values_kernel<16>, dim3(units * NS), dim3(256), 0, st, p);
  hipLaunchKernelGGL(decode_combine_kernel, dim3(units), dim3(256), 0, st, p);
  return launch_status();
}

extern "C" int hsg_ring_decode_rope(const void* q_raw, int64_t q_row, int64_t q_head, const float* q_w1, float q_eps,
                                    const void* k_raw, int64_t k_row, int64_t k_head, const float* k_w1, float k_eps,
                                    const int64_t* pos, const float* inv_freq, int32_t rot, void* k_out,
                                    int64_t ko_row, void* ring_k, void* ring_v, int64_t ring_rows, int32_t window,
                                    const void* new_v, int64_t nv_row, int64_t nv_head, const void* gate,
                                    int64_t g_row, int64_t g_head, int64_t g_group, int64_t g_off,
                                    const int64_t* ring_pos, const int64_t* slots, const int64_t* starts,
                                    const int64_t* lens, const int64_t* offsets, int32_t n_rows, int32_t hkv,
                                    int32_t groups, int32_t head_dim, float scale, int32_t write_ring, void* out,
                                    int64_t o_row, int64_t o_head, int64_t o_group, void* workspace,
                                    size_t workspace_bytes, void* stream) {
  using namespace hsg;
  if (n_rows < 0 || hkv <= 0 || groups <= 0 || ring_rows <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  if (!q_raw || !q_w1 || !k_raw || !k_w1 || !pos || !inv_freq || !k_out || !ring_k || !ring_v || !new_v ||
      !ring_pos || !slots || !starts || !lens || !offsets || !out || !workspace)
    return HSG_ERR_ARG;
  if (head_dim != D || rot != 64 || window <= 0 || window > W_MAX || window % KB != 0 || groups > G_MAX ||
      workspace_bytes < hsg_ring_decode_workspace_bytes(n_rows, hkv, groups, window))
    return HSG_ERR_SHAPE;
  const int64_t s8[] = {q_row, q_head, k_row, k_head, ko_row, nv_row, nv_head, g_row, g_head, g_group, g_off, o_row,
                        o_head, o_group};
  for (int64_t v : s8)
    if (v % 4) return HSG_ERR_ALIGN;
  if (!aligned(q_raw, 8) || !aligned(k_raw, 8) || !aligned(k_out, 8) || !aligned(q_w1, 16) || !aligned(k_w1, 16) ||
      !aligned(ring_k, 16) || !aligned(ring_v, 16) || !aligned(new_v, 8) || !aligned(out, 8) ||
      (gate && !aligned(gate, 8)) || !aligned(workspace, 16))
    return HSG_ERR_ALIGN;
  DecParams p{};
  p.q = static_cast<const uint16_t*>(q_raw);   // not read: the scores kernel takes q_raw
  p.ring_k = static_cast<uint16_t*>(ring_k); p.ring_v = static_cast<uint16_t*>(ring_v);
  p.ring_rows = ring_rows; p.W = window;
  p.new_k = static_cast<const uint16_t*>(k_out); p.nk_sl = ko_row; p.nk_sh = D;   // the combine's ring write
  p.new_v = static_cast<const uint16_t*>(new_v); p.nv_sl = nv_row; p.nv_sh = nv_head;
  p.gate = static_cast<const uint16_t*>(gate);
  p.g_sl = g_row; p.g_sh = g_head; p.g_sg = g_group; p.g_off = g_off;
  p.ring_pos = ring_pos; p.slots = slots; p.starts = starts; p.lens = lens; p.offsets = offsets;
  p.hkv = hkv; p.G = groups; p.scale = scale; p.write_ring = write_ring;
  p.out = static_cast<uint16_t*>(out); p.o_sl = o_row; p.o_sh = o_head; p.o_sg = o_group;
  p.ws = static_cast<float*>(workspace);
  p.unit = unit_floats(groups, window);
  p.sc_stride = window + KB;
  p.q_raw = static_cast<const uint16_t*>(q_raw); p.qr_sl = q_row; p.qr_sh = q_head;
  p.k_raw = static_cast<const uint16_t*>(k_raw); p.kr_sl = k_row; p.kr_sh = k_head;
  p.q_w1 = q_w1; p.k_w1 = k_w1; p.q_eps = q_eps; p.k_eps = k_eps;
  p.pos = pos; p.inv_freq = inv_freq; p.rot = rot;
  p.k_out = static_cast<uint16_t*>(k_out);
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const unsigned units = (unsigned)(n_rows * hkv);
  hipLaunchKernelGGL(decode_scores_kernel<true>, dim3(units * NS), dim3(256), 0, st, p);
  if (groups <= 4) hipLaunchKernelGGL(decode_values_kernel<4>, dim3(units * NS), dim3(256), 0, st, p);
  else if (groups <= 8) hipLaunchKernelGGL(decode_values_kernel<8>, dim3(units * NS), dim3(256), 0, st, p);
  else hipLaunchKernelGGL(decode_values_kernel<16>, dim3(units * NS), dim3(256), 0, st, p);
  hipLaunchKernelGGL(decode_combine_kernel, dim3(units), dim3(256), 0, st, p);
  return launch_status();
}

// ---------------------------------------------------------------------------------------------------------
// Allocation-free variant: the split-K workspace is a static device array of the library, one copy per GPU,
// held until the process ends. Host code never passes `scratch` itself to a kernel (on the host that name is a
// stand-in, not a device address): the device address of each GPU's copy is looked up once per device with
// hipGetSymbolAddress and kept in scratch_ptr[device].
static __device__ __align__(256) unsigned char scratch[HSG_RING_DECODE_SCRATCH_BYTES];

namespace {
constexpr int kMaxDevices = 64;
std::mutex scratch_mu;
void* scratch_ptr[kMaxDevices] = {};

// device address of the current device's scratch (looked up on the first call made on that device)
int current_scratch(void** out) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return HSG_ERR_ARG;
  std::lock_guard<std::mutex> lock(scratch_mu);
  if (scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess) return (int)e;
    if (p == nullptr) return HSG_ERR_ARG;
    scratch_ptr[dev] = p;
  }
  *out = scratch_ptr[dev];
  return HSG_OK;
}
}  // namespace

extern "C" int hsg_ring_decode_noalloc(const void* q, int64_t q_sn, int64_t q_sl, int64_t q_sh, int64_t q_sg,
                                       void* ring_k, void* ring_v, int64_t ring_rows, int32_t window,
                                       const void* new_k, int64_t nk_sn, int64_t nk_sl, int64_t nk_sh,
                                       const void* new_v, int64_t nv_sn, int64_t nv_sl, int64_t nv_sh,
                                       const void* gate, int64_t g_sn, int64_t g_sl, int64_t g_sh, int64_t g_sg,
                                       int64_t g_off, const int64_t* ring_pos, const int64_t* slots,
                                       const int64_t* starts, const int64_t* lens, const int64_t* offsets,
                                       int32_t n_rows, int32_t hkv, int32_t groups, int32_t head_dim, float scale,
                                       int32_t write_ring, void* out, int64_t o_sn, int64_t o_sl, int64_t o_sh,
                                       int64_t o_sg, void* stream) {
  if (n_rows < 0 || hkv <= 0 || groups <= 0 || ring_rows <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  // the scratch bounds only the split-K path above 8 query heads per kv head (up to 8 it runs for at most
  // HSG_RING_DECODE_SPLIT_UNITS rows x kv heads, which the scratch always holds)
  if (groups > 8 &&
      hsg_ring_decode_workspace_bytes(n_rows, hkv, groups, window) > (size_t)HSG_RING_DECODE_SCRATCH_BYTES)
    return HSG_ERR_SHAPE;
  void* ws = nullptr;
  const int rc = current_scratch(&ws);
  if (rc != HSG_OK) return rc;
  // the fused kernel does not touch the workspace; the split-K kernels write every workspace word they read
  // (scores of visible blocks, every block maximum, every split's partial sums), so nothing left by an earlier call
  // is read and nothing needs clearing
  return hsg_ring_decode(q, q_sn, q_sl, q_sh, q_sg, ring_k, ring_v, ring_rows, window, new_k, nk_sn, nk_sl, nk_sh,
                         new_v, nv_sn, nv_sl, nv_sh, gate, g_sn, g_sl, g_sh, g_sg, g_off, ring_pos, slots, starts,
                         lens, offsets, n_rows, hkv, groups, head_dim, scale, write_ring, out, o_sn, o_sl, o_sh,
                         o_sg, ws, (size_t)HSG_RING_DECODE_SCRATCH_BYTES, stream);
}
