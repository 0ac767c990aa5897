// Window-W GQA ring attention (decode and short ticks) for gfx950.
//
// Contract: src/hs_guard/engine/ring_attention_kernel.py:7-26 (torch reference) with the v8 epilogue of
// src/hs_guard/engine/fused_kernels.py:341-355 (bf16 output times bf16(sigmoid(gate)), in-place ring write).
//
// Mapping: one workgroup of NW = 4 waves per (row, kv head); the workgroup owns that (slot, kv head)'s
// ring, so the ring write at the end cannot race with any read. The W ring columns are split across the
// waves (split-K inside the workgroup: each wave keeps its own max / sum / accumulator and the four are
// merged through LDS), and the tick's new keys are dealt round-robin to the waves. Queries are processed
// four rows at a time: the G = Hq/Hkv query heads of one token l share the token's position, so the
// window predicate is uniform over the four rows and masked columns are skipped without reading K or V.
//   Scores: 16 lanes per key (each a contiguous 32-byte slice of the 512-byte key row, so 16 lanes read
//   one row), 4 keys per wave instruction, butterfly over the 16 lanes.
//   Values: each lane owns 4 of the 256 dims, one coalesced 512-byte row per key.
#include <math.h>

#include "hsg_common.h"

namespace hsg {
namespace {

constexpr int D = 256;
constexpr int NW = 4;
constexpr int W_MAX = 512;
constexpr int LB_MAX = 64;
constexpr int CW_MAX = W_MAX / NW;
constexpr int NEW_MAX = LB_MAX / NW;
constexpr int COLS_MAX = CW_MAX + NEW_MAX;

struct RingParams {
  const uint16_t* q; int64_t q_sn, q_sl, q_sh, q_sg;
  uint16_t* ring_k; uint16_t* ring_v; int64_t ring_rows; int W;
  const uint16_t* new_k; int64_t nk_sn, nk_sl, nk_sh;
  const uint16_t* new_v; int64_t nv_sn, nv_sl, nv_sh;
  const uint16_t* gate; int64_t g_sn, g_sl, g_sh, g_sg, g_off;
  const int64_t* ring_pos; const int64_t* slots; const int64_t* starts; const int64_t* lens;
  const int64_t* offsets;
  int lb, hkv, G;
  float scale;
  int write_ring;
  uint16_t* out; int64_t o_sn, o_sl, o_sh, o_sg;
};

__device__ __forceinline__ float sum16(float x) {
  x = xor_add<1>(x); x = xor_add<2>(x); x = xor_add<4>(x); x = xor_add<8>(x);
  return x;
}

__global__ __launch_bounds__(NW * 64) void ring_attn_kernel(const RingParams p) {
  __shared__ float sc[NW][4][COLS_MAX];
  __shared__ float accs[NW][4][D];
  __shared__ float mls[NW][4][2];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = blockIdx.x / p.hkv;
  const int h = blockIdx.x - n * p.hkv;
  const int64_t slot = p.slots[n];
  const int64_t start = p.starts[n];
  int64_t len = p.lens[n];
  const bool padded = p.offsets == nullptr;
  if (slot < 0 || slot >= p.ring_rows || len < 0 || len > LB_MAX) len = 0;  // > LB_MAX: rejected row
  if (padded && len > p.lb) len = p.lb;
  const int steps = padded ? p.lb : (int)len;          // output steps written for this row
  const int64_t base_tok = padded ? 0 : p.offsets[n];
  const int64_t q_row = padded ? n * p.q_sn : base_tok * p.q_sl;
  const int64_t nk_row = padded ? n * p.nk_sn : base_tok * p.nk_sl;
  const int64_t nv_row = padded ? n * p.nv_sn : base_tok * p.nv_sl;
  const int64_t g_row = padded ? n * p.g_sn : base_tok * p.g_sl;
  const int64_t o_row = padded ? n * p.o_sn : base_tok * p.o_sl;
  const int W = p.W;
  const int cw = W / NW;
  const int nnew = (int)len;                            // valid new keys (j < len)
  const int64_t ring_base = ((slot * p.hkv + h) * (int64_t)(W + 1)) * D;
  const int64_t* rpos = p.ring_pos + slot * (int64_t)(W + 1);
  const int sub = lane & 15;
  const int ks = lane >> 4;
  const int groups4 = (p.G + 3) >> 2;

  for (int quad = 0; quad < steps * groups4; ++quad) {
    const int l = quad / groups4;
    const int g0 = (quad - l * groups4) * 4;
    const bool q_valid = l < len;
    const int64_t qpos = start + l;
    if (!q_valid) {  // no visible key: output 0 (times the gate is still 0)
      for (int e = tid; e < 4 * (D / 4); e += NW * 64) {
        const int i = e / (D / 4);
        const int d = (e - i * (D / 4)) * 4;
        if (g0 + i < p.G) {
          const float zero[4] = {0.f, 0.f, 0.f, 0.f};
          store4_bf16(p.out + o_row + l * p.o_sl + h * p.o_sh + (g0 + i) * p.o_sg + d, zero);
        }
      }
      continue;
    }
    // ---- queries of the quad: lane holds dims [16 sub, 16 sub + 16) of each of the 4 rows ----
    float qf[4][16];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (g0 + i < p.G) {
        const uint16_t* qp = p.q + q_row + l * p.q_sl + h * p.q_sh + (g0 + i) * p.q_sg + sub * 16;
        load8_bf16(qp, qf[i]);
        load8_bf16(qp + 8, qf[i] + 8);
      } else {
#pragma unroll
        for (int e = 0; e < 16; ++e) qf[i][e] = 0.f;
      }
    }
    // ---- pass 1: scores of this wave's columns (ring slice, then its share of the new keys) ----
    const int c0 = wave * cw;
    const int my_new = nnew > wave ? (nnew - wave + NW - 1) / NW : 0;
    const int ncols = cw + my_new;
    for (int vb = 0; vb < ncols; vb += 4) {
      const int vi = vb + ks;
      bool ok = false;
      const uint16_t* kp = nullptr;
      if (vi < cw) {
        const int64_t kpos = rpos[c0 + vi];
        ok = kpos >= 0 && kpos <= qpos && kpos > qpos - W;
        kp = p.ring_k + ring_base + (int64_t)(c0 + vi) * D;
      } else if (vi < ncols) {
        const int j = wave + (vi - cw) * NW;
        const int64_t kpos = start + j;  // j < len by construction
        ok = kpos <= qpos && kpos > qpos - W;
        kp = p.new_k + nk_row + j * p.nk_sl + h * p.nk_sh;
      }
      float s[4] = {0.f, 0.f, 0.f, 0.f};
      if (ok) {
        float kf[16];
        load8_bf16(kp + sub * 16, kf);
        load8_bf16(kp + sub * 16 + 8, kf + 8);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
#pragma unroll
          for (int e = 0; e < 16; ++e) s[i] += qf[i][e] * kf[e];
        }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) s[i] = sum16(s[i]);
      if (sub == 0 && vi < ncols) {
#pragma unroll
        for (int i = 0; i < 4; ++i) sc[wave][i][vi] = ok ? s[i] * p.scale : -INFINITY;
      }
    }
    // ---- wave-local softmax statistics (LDS written by this wave only; wave-synchronous) ----
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    float m[4], lsum[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float mx = -INFINITY;
      for (int vi = lane; vi < ncols; vi += 64) mx = fmaxf(mx, sc[wave][i][vi]);
      m[i] = wave_max(mx);
      float sm = 0.f;
      for (int vi = lane; vi < ncols; vi += 64) {
        const float sv = sc[wave][i][vi];
        const float pv = (m[i] == -INFINITY || sv == -INFINITY) ? 0.f : expf(sv - m[i]);
        sc[wave][i][vi] = pv;
        sm += pv;
      }
      lsum[i] = wave_sum(sm);
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
    // ---- pass 2: P V over the same columns; lane owns dims [4 lane, 4 lane + 4) ----
    float acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
#pragma unroll
      for (int e = 0; e < 4; ++e) acc[i][e] = 0.f;
    }
    for (int vi = 0; vi < ncols; ++vi) {
      const float p0 = sc[wave][0][vi], p1 = sc[wave][1][vi], p2 = sc[wave][2][vi], p3 = sc[wave][3][vi];
      if (p0 == 0.f && p1 == 0.f && p2 == 0.f && p3 == 0.f) continue;
      const uint16_t* vp;
      if (vi < cw) {
        vp = p.ring_v + ring_base + (int64_t)(c0 + vi) * D;
      } else {
        const int j = wave + (vi - cw) * NW;
        vp = p.new_v + nv_row + j * p.nv_sl + h * p.nv_sh;
      }
      float vf[4];
      load4_bf16(vp + lane * 4, vf);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        acc[0][e] += p0 * vf[e];
        acc[1][e] += p1 * vf[e];
        acc[2][e] += p2 * vf[e];
        acc[3][e] += p3 * vf[e];
      }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      *reinterpret_cast<float4*>(&accs[wave][i][lane * 4]) = make_float4(acc[i][0], acc[i][1], acc[i][2], acc[i][3]);
      if (lane == 0) {
        mls[wave][i][0] = m[i];
        mls[wave][i][1] = lsum[i];
      }
    }
    __syncthreads();
    // ---- merge the four waves, normalise, gate, store ----
    {
      const int i = tid >> 6;
      const int d = (tid & 63) * 4;
      if (g0 + i < p.G) {
        float mmax = -INFINITY;
#pragma unroll
        for (int w = 0; w < NW; ++w) mmax = fmaxf(mmax, mls[w][i][0]);
        float num[4] = {0.f, 0.f, 0.f, 0.f};
        float den = 0.f;
        if (mmax != -INFINITY) {
#pragma unroll
          for (int w = 0; w < NW; ++w) {
            const float mw = mls[w][i][0];
            const float f = mw == -INFINITY ? 0.f : expf(mw - mmax);
            den += f * mls[w][i][1];
            const float4 a4 = *reinterpret_cast<const float4*>(&accs[w][i][d]);
            num[0] += f * a4.x; num[1] += f * a4.y; num[2] += f * a4.z; num[3] += f * a4.w;
          }
        }
        float y[4];
#pragma unroll
        for (int e = 0; e < 4; ++e) y[e] = den > 0.f ? rbf(num[e] / den) : 0.f;
        if (p.gate != nullptr) {
          float gt[4];
          load4_bf16(p.gate + g_row + l * p.g_sl + h * p.g_sh + (g0 + i) * p.g_sg + p.g_off + d, gt);
#pragma unroll
          for (int e = 0; e < 4; ++e) y[e] = y[e] * rbf(1.0f / (1.0f + expf(-gt[e])));
        }
        store4_bf16(p.out + o_row + l * p.o_sl + h * p.o_sh + (g0 + i) * p.o_sg + d, y);
      }
    }
    __syncthreads();
  }

  // ---- in-place ring write of this tick's valid keys/values (all reads of this ring are done) ----
  if (p.write_ring && len > 0) {
    for (int e = tid; e < nnew * (D / 4); e += NW * 64) {
      const int j = e / (D / 4);
      const int d = (e - j * (D / 4)) * 4;
      const int64_t col = (start + j) % W;
      const int64_t dst = ring_base + col * D + d;
      *reinterpret_cast<uint2*>(p.ring_k + dst) =
          *reinterpret_cast<const uint2*>(p.new_k + nk_row + j * p.nk_sl + h * p.nk_sh + d);
      *reinterpret_cast<uint2*>(p.ring_v + dst) =
          *reinterpret_cast<const uint2*>(p.new_v + nv_row + j * p.nv_sl + h * p.nv_sh + d);
    }
  }
}

}  // namespace
}  // namespace hsg

extern "C" int hsg_ring_attention(const void* q, int64_t q_sn, int64_t q_sl, int64_t q_sh, int64_t q_sg,
                                  void* ring_k, void* ring_v, int64_t ring_rows, int32_t window,
                                  const void* new_k, int64_t nk_sn, int64_t nk_sl, int64_t nk_sh,
                                  const void* new_v, int64_t nv_sn, int64_t nv_sl, int64_t nv_sh,
                                  const void* gate, int64_t g_sn, int64_t g_sl, int64_t g_sh, int64_t g_sg,
                                  int64_t g_off, const int64_t* ring_pos, const int64_t* slots,
                                  const int64_t* starts, const int64_t* lens, const int64_t* offsets,
                                  int32_t n_rows, int32_t lb, int32_t hkv, int32_t groups, int32_t head_dim,
                                  float scale, int32_t write_ring, void* out, int64_t o_sn, int64_t o_sl,
                                  int64_t o_sh, int64_t o_sg, void* stream) {
  using namespace hsg;
  if (n_rows < 0 || lb <= 0 || hkv <= 0 || groups <= 0 || ring_rows <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  if (!q || !ring_k || !ring_v || !new_k || !new_v || !ring_pos || !slots || !starts || !lens || !out)
    return HSG_ERR_ARG;
  if (head_dim != D || window <= 0 || window > W_MAX || window % (4 * NW) != 0 || lb > LB_MAX) return HSG_ERR_SHAPE;
  if (write_ring && lb > window) return HSG_ERR_SHAPE;  // two steps of one tick would share a ring column
  const int64_t s16[] = {q_sn, q_sl, q_sh, q_sg};
  for (int64_t s : s16)
    if (s % 8) return HSG_ERR_ALIGN;
  const int64_t s4[] = {nk_sn, nk_sl, nk_sh, nv_sn, nv_sl, nv_sh, g_sn, g_sl, g_sh, g_sg, g_off, o_sn, o_sl, o_sh, o_sg};
  for (int64_t s : s4)
    if (s % 4) return HSG_ERR_ALIGN;
  if (!aligned(q, 16) || !aligned(ring_k, 16) || !aligned(ring_v, 16) || !aligned(new_k, 16) ||
      !aligned(new_v, 8) || !aligned(out, 8) || (gate && !aligned(gate, 8)))
    return HSG_ERR_ALIGN;
  RingParams p{};
  p.q = static_cast<const uint16_t*>(q); p.q_sn = q_sn; p.q_sl = q_sl; p.q_sh = q_sh; p.q_sg = q_sg;
  p.ring_k = static_cast<uint16_t*>(ring_k); p.ring_v = static_cast<uint16_t*>(ring_v);
  p.ring_rows = ring_rows; p.W = window;
  p.new_k = static_cast<const uint16_t*>(new_k); p.nk_sn = nk_sn; p.nk_sl = nk_sl; p.nk_sh = nk_sh;
  p.new_v = static_cast<const uint16_t*>(new_v); p.nv_sn = nv_sn; p.nv_sl = nv_sl; p.nv_sh = nv_sh;
  p.gate = static_cast<const uint16_t*>(gate);
  p.g_sn = g_sn; p.g_sl = g_sl; p.g_sh = g_sh; p.g_sg = g_sg; p.g_off = g_off;
  p.ring_pos = ring_pos; p.slots = slots; p.starts = starts; p.lens = lens; p.offsets = offsets;
  p.lb = lb; p.hkv = hkv; p.G = groups; p.scale = scale; p.write_ring = write_ring;
  p.out = static_cast<uint16_t*>(out); p.o_sn = o_sn; p.o_sl = o_sl; p.o_sh = o_sh; p.o_sg = o_sg;
  hipLaunchKernelGGL(ring_attn_kernel, dim3((unsigned)(n_rows * hkv)), dim3(NW * 64), 0,
                     reinterpret_cast<hipStream_t>(stream), p);
  return launch_status();
}
