// Window-W GQA ring attention (decode, short ticks and 64-token window fills) for gfx950 on MFMA.
//
// Contract: src/hs_guard/engine/ring_attention_kernel.py:7-26 (torch reference) with the v8 kernel's
// numerics and epilogue (src/hs_guard/engine/fused_kernels.py:288-356): keys in blocks of 32 (the W ring
// columns in order, then the tick's new keys), a running max per query row, probabilities rounded to bf16
// in the P.V product and summed in fp32, output / sum rounded to bf16, times bf16(sigmoid(gate)); the
// tick's keys/values are written into the ring in place after every read.
//
// Mapping: query rows r = l*G + g (token l, q group g) of one (row, kv head) form 16-row tiles; one
// workgroup (4 waves) per (row, kv head, query group qg), wave w taking tile 4*qg + w, so a 64-step row
// spreads over several workgroups that stream the same ring in parallel. The in-place ring write is a second
// launch (ring_write_kernel) after all reads. All key positions of the ring and the tick go to LDS first, and
// fills (64 keys) whose positions are outside every query's window of the workgroup are skipped. Per fill the
// workgroup stages K and V row-major in LDS from registers loaded during the previous fill (each load
// instruction of a wave reads two whole 512-byte key rows); then each wave runs on v_mfma_f32_16x16x32_bf16
//   S^T[key, m] = K . Q^T   (A = K rows from LDS, B = Q from registers; 2 key tiles x 8 d-steps)
// for both of the fill's 32-key softmax blocks first (four independent accumulation chains instead of two:
// the fill's critical path is this chain, then the softmax, then P.V), and then, block by block,
//   O^T[d, m] += V^T . P^T  (A = V^T by LDS transpose reads of the row-major V, B = P straight from the S^T
//                            accumulators: the k order of the product is the lane's own key order, so P
//                            never leaves registers)
// The S^T accumulator layout puts one query row per lane column, so the running max / sum and the O^T
// rescale are per-lane scalars plus a 2-step butterfly (lane xor 16, 32).
#include <math.h>

#include "hsg_common.h"

namespace hsg {
namespace {

constexpr int D = 256;
constexpr int NW = 4;
constexpr int KB = 32;                 // keys per softmax block (the reference's BN)
constexpr int SB = 2;                  // softmax blocks staged per LDS fill
constexpr int KF = KB * SB;            // keys per LDS fill
constexpr int W_MAX = 512;
constexpr int LB_MAX = 64;
constexpr int KS_STRIDE = D + 8;       // bf16 per K or V row in LDS (16-byte pad)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(4))) float f32x4;

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
  int min_len;
  int qgroups;      // workgroups per (row, kv head): groups of NW 16-row query tiles
  uint16_t* out; int64_t o_sn, o_sl, o_sh, o_sg;
};

__device__ __forceinline__ bf16x8 as_bf16x8(uint4 w) { return __builtin_bit_cast(bf16x8, w); }

constexpr int KP_NONE = -(1 << 30);

// exp of the softmax argument on the hardware exp2 (v_exp_f32): exp(x) = 2^(x log2 e). The reference kernel
// takes tl.exp, Triton's fast exponential, here too (src/hs_guard/engine/fused_kernels.py:318-319,335-336).
__device__ __forceinline__ float exp_fast(float x) { return __builtin_amdgcn_exp2f(x * 1.4426950408889634f); }

typedef __attribute__((ext_vector_type(4))) short s16x4_;

// LDS transpose read (ds_read_b64_tr_b16): within each group of 16 lanes, lane 4q + e receives element e of
// the 4-element (8-byte) vectors addressed by lanes q, q + 4, q + 8, q + 12 of its group. With V row-major
// ([key][dim]), lane s of a group addressing key row r0 + (s >> 2), dims c0 + 4 (s & 3) .. +3 receives dim
// c0 + s of keys r0 .. r0 + 3: the A operand of O^T += V^T . P^T.
__device__ __forceinline__ uint2 ld_tr4(const uint16_t* p) {
  return __builtin_bit_cast(uint2, __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4_*)(p)));
}

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return (uint32_t)f2bf(lo) | ((uint32_t)f2bf(hi) << 16);
}

__global__ __launch_bounds__(NW * 64, 2) void ring_attn_mfma_kernel(const RingParams p) {
  __shared__ __align__(16) uint16_t Ks[KF * KS_STRIDE];
  __shared__ __align__(16) uint16_t Vs[KF * KS_STRIDE];
  // key position - start (the row's first new position), clamped to [-2W-1, 2W+1]; KP_NONE for an empty
  // column: ring columns [0, W), then the tick's new keys
  __shared__ int kp_all[W_MAX + LB_MAX];
  __shared__ uint32_t wave_mask[NW];           // per wave: bit f set if fill f has a key visible to the group

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  // query group slowest: consecutive workgroups (which the dispatcher deals round-robin over the 8 XCDs)
  // take consecutive (row, kv head) pairs, so the live workgroups of a short-row tick spread over all XCDs
  const int n_pairs = gridDim.x / p.qgroups;
  const int qg = blockIdx.x / n_pairs;
  const int nh = blockIdx.x - qg * n_pairs;
  const int n = nh / p.hkv;
  const int h = nh - n * p.hkv;
  const int64_t slot = p.slots[n];
  const int64_t start = p.starts[n];
  int64_t len = p.lens[n];
  const bool padded = p.offsets == nullptr;
  if (slot < 0 || slot >= p.ring_rows || len < 0 || len > (padded ? LB_MAX : p.lb)) len = 0;  // rejected row
  if (padded && len > p.lb) len = p.lb;
  if (!padded && len < p.min_len) return;              // left to another kernel (single-step rows: split-K)
  const int steps = padded ? p.lb : (int)len;          // output steps written for this row
  const int64_t base_tok = padded ? 0 : p.offsets[n];
  const int64_t q_row = padded ? n * p.q_sn : base_tok * p.q_sl;
  const int64_t nk_row = padded ? n * p.nk_sn : base_tok * p.nk_sl;
  const int64_t nv_row = padded ? n * p.nv_sn : base_tok * p.nv_sl;
  const int64_t g_row = padded ? n * p.g_sn : base_tok * p.g_sl;
  const int64_t o_row = padded ? n * p.o_sn : base_tok * p.o_sl;
  const int W = p.W;
  const int G = p.G;
  const int64_t ring_base = ((slot * p.hkv + h) * (int64_t)(W + 1)) * D;
  const int64_t* rpos = p.ring_pos + slot * (int64_t)(W + 1);
  const int M = G * steps;                              // query rows of this (row, kv head)
  const int QT = (M + 15) >> 4;                         // 16-row tiles
  const int q4 = lane >> 4;                             // lane group: keys 4*q4 .., dims 8*q4 ..
  const int mcol = lane & 15;                           // the lane's query row within its tile
  const int n_ring_blocks = len > 0 ? W / KB : 0;
  const int n_new_blocks = (int)((len + KB - 1) / KB);

  if (qg * NW < QT) {
    const int tile = qg * NW + wave;
    const bool has_tile = tile < QT;
    // ---- this lane's query row ----
    const int r = tile * 16 + mcol;
    const int l_tok = r / G;
    const int gq = r - l_tok * G;
    const bool row_ok = has_tile && r < M;
    const bool q_valid = row_ok && l_tok < len;
    bf16x8 qb[D / 32];
#pragma unroll
    for (int ks = 0; ks < D / 32; ++ks) {
      uint4 w = make_uint4(0u, 0u, 0u, 0u);
      if (q_valid)
        w = *reinterpret_cast<const uint4*>(p.q + q_row + l_tok * p.q_sl + h * p.q_sh + gq * p.q_sg + 32 * ks + 8 * q4);
      qb[ks] = as_bf16x8(w);
    }
    // positions covered by this query group (all waves), for skipping whole key blocks
    const int r_lo = qg * NW * 16;
    const int r_hi = min(M, (qg + 1) * NW * 16) - 1;
    const int64_t qpos_lo = start + r_lo / G;
    const int64_t qpos_hi = start + min((int64_t)(r_hi / G), len - 1);
    float m_run = -INFINITY, l_run = 0.f;
    f32x4 O[D / 16];
#pragma unroll
    for (int t = 0; t < D / 16; ++t) O[t] = (f32x4){0.f, 0.f, 0.f, 0.f};

    // Fills: n_ring_fills of up to SB ring blocks, then the new-key blocks in fills of up to SB. Every key
    // position goes to LDS in one round trip and the fills no query of this group sees are skipped; the
    // next visible fill's K and V are loaded into registers while the current one is computed.
    const int n_ring_fills = (n_ring_blocks + SB - 1) / SB;
    const int n_fills = n_ring_fills + (n_new_blocks + SB - 1) / SB;
    uint32_t my_mask = 0u;
    for (int c = tid; c < W + n_new_blocks * KB; c += NW * 64) {
      int64_t kpos;
      int f;
      if (c < W) {
        kpos = c < n_ring_blocks * KB ? rpos[c] : -1;
        f = c / KF;
      } else {
        const int j = c - W;
        kpos = j < len ? start + j : -1;
        f = n_ring_fills + j / KF;
      }
      const int64_t rel = kpos - start;
      kp_all[c] = kpos < 0 ? KP_NONE : (int)(rel < -2 * W - 1 ? -2 * W - 1 : rel > 2 * W + 1 ? 2 * W + 1 : rel);
      if (kpos >= 0 && kpos <= qpos_hi && kpos > qpos_lo - W) my_mask |= 1u << f;
    }
    // OR over the workgroup: wave butterfly, then one word per wave through LDS
    for (int o = 1; o < 64; o <<= 1) my_mask |= (uint32_t)__shfl_xor((int)my_mask, o, 64);
    if (lane == 0) wave_mask[wave] = my_mask;
    __syncthreads();
    const uint32_t fmask = wave_mask[0] | wave_mask[1] | wave_mask[2] | wave_mask[3];
    auto fill_geom = [&](int f, bool& is_ring, int& c0, int& nb) {
      is_ring = f < n_ring_fills;
      const int b0 = is_ring ? f * SB : (f - n_ring_fills) * SB;
      nb = is_ring ? min(SB, n_ring_blocks - b0) : min(SB, n_new_blocks - b0);
      c0 = b0 * KB;   // ring column or new-key index of the fill's first key
    };
    // Thread t holds dims 8 (t % 32) .. +7 of keys t / 32 + 8 i (i < 8) of K and of V: every load instruction
    // of a wave reads two whole 512-byte key rows. Keys past the fill's valid ones load a clamped valid row
    // and are zeroed when staged.
    u32x4 kr[8], vr[8];
    auto prefetch = [&](int f) {
      bool is_ring; int c0, nb;
      fill_geom(f, is_ring, c0, nb);
      const int nkeys = nb * KB;
      const int dcol = 8 * (tid & 31);
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int key = (tid >> 5) + 8 * i;
        const uint16_t* ksrc;
        const uint16_t* vsrc;
        if (is_ring) {
          const int64_t off = ring_base + (int64_t)(c0 + min(key, nkeys - 1)) * D + dcol;
          ksrc = p.ring_k + off;
          vsrc = p.ring_v + off;
        } else {
          const int64_t j = min(c0 + key, (int)len - 1);
          ksrc = p.new_k + nk_row + j * p.nk_sl + h * p.nk_sh + dcol;
          vsrc = p.new_v + nv_row + j * p.nv_sl + h * p.nv_sh + dcol;
        }
        // nontemporal, as the decode kernel's ring reads: a step's mixed tick ran 0.35 % faster (two A/B pairs
        // on MI355X), the rings no longer displacing what the neighbouring kernels reuse
        kr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(ksrc));
        vr[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(vsrc));
      }
    };
    auto next_fill = [&](int f) {   // first visible fill after f (n_fills if none)
      const uint32_t rest = f + 1 < 32 ? (fmask >> (f + 1)) : 0u;
      return rest ? f + 1 + __builtin_ctz(rest) : n_fills;
    };
    int fcur = next_fill(-1);
    if (fcur < n_fills) prefetch(fcur);
    for (; fcur < n_fills; fcur = next_fill(fcur)) {
      bool is_ring; int c0, nb;
      fill_geom(fcur, is_ring, c0, nb);
      const int nkeys = nb * KB;
      const int kbase = is_ring ? c0 : W + c0;   // the fill's first key in kp_all
      __syncthreads();  // the previous fill's LDS reads are done
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int key = (tid >> 5) + 8 * i;
        const bool live = key < nkeys && (is_ring || c0 + key < len);
        const int o = key * KS_STRIDE + 8 * (tid & 31);
        *reinterpret_cast<u32x4*>(&Ks[o]) = live ? kr[i] : (u32x4){0u, 0u, 0u, 0u};
        *reinterpret_cast<u32x4*>(&Vs[o]) = live ? vr[i] : (u32x4){0u, 0u, 0u, 0u};
      }
      const int fnext = next_fill(fcur);
      if (fnext < n_fills) prefetch(fnext);
      __syncthreads();
      if (!has_tile) continue;
      // ---- S^T = K . Q^T for both softmax blocks of the fill first (four independent accumulation chains) ----
      f32x4 Sall[SB][2];
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        if (sb < nb) {
#pragma unroll
          for (int kt = 0; kt < 2; ++kt) {
            f32x4 acc = {0.f, 0.f, 0.f, 0.f};
            const uint16_t* krow = &Ks[(sb * KB + 16 * kt + mcol) * KS_STRIDE + 8 * q4];
#pragma unroll
            for (int ks = 0; ks < D / 32; ++ks) {
              const bf16x8 a = as_bf16x8(*reinterpret_cast<const uint4*>(krow + 32 * ks));
              acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, qb[ks], acc, 0, 0, 0);
            }
            Sall[sb][kt] = acc;
          }
        }
      }
#pragma unroll
      for (int sb = 0; sb < SB; ++sb) {
        if (sb >= nb) break;
        const int kb = sb * KB;   // softmax block within the fill
        const f32x4 S[2] = {Sall[sb][0], Sall[sb][1]};
        // ---- mask, online softmax over the block (the lane's 8 keys: 4 q4 + i and 16 + 4 q4 + i) ----
        float s[8];
        float bmax = -INFINITY;
#pragma unroll
        for (int kt = 0; kt < 2; ++kt) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const int rel = kp_all[kbase + kb + 16 * kt + 4 * q4 + i];
            const bool ok = q_valid && rel <= l_tok && rel > l_tok - W;   // KP_NONE fails the second
            const float v = ok ? S[kt][i] * p.scale : -INFINITY;
            s[4 * kt + i] = v;
            bmax = fmaxf(bmax, v);
          }
        }
        bmax = max_pair32(max_pair16(bmax));   // over q4 (lane xor 16, 32)
        const float m_new = fmaxf(m_run, bmax);
        const float m_safe = m_new == -INFINITY ? 0.f : m_new;
        const float alpha = exp_fast(m_run - m_safe);   // exp(-inf) = 0 before the first visible key
        float psum = 0.f;
        uint32_t pk[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float p0 = exp_fast(s[2 * i] - m_safe);
          const float p1 = exp_fast(s[2 * i + 1] - m_safe);
          psum += p0 + p1;
          pk[i] = pack_bf16(p0, p1);
        }
        psum = add_xor32(add_xor16(psum));
        l_run = l_run * alpha + psum;
        m_run = m_new;
        const bf16x8 pb = as_bf16x8(make_uint4(pk[0], pk[1], pk[2], pk[3]));
        // ---- O^T += V^T . P^T over the block's 32 keys, in the lane's key order ----
#pragma unroll
        for (int t = 0; t < D / 16; ++t) {
          // dim 16 t + mcol of keys kb + 4 q4 .. +3 and kb + 16 + 4 q4 .. +3 (the lane's key order of P)
          const uint16_t* vsrc = &Vs[(kb + 4 * q4 + (mcol >> 2)) * KS_STRIDE + 16 * t + 4 * (mcol & 3)];
          const uint2 lo = ld_tr4(vsrc);
          const uint2 hi = ld_tr4(vsrc + 16 * KS_STRIDE);
          const bf16x8 a = as_bf16x8(make_uint4(lo.x, lo.y, hi.x, hi.y));
          f32x4 o = O[t];
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] *= alpha;
          O[t] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, pb, o, 0, 0, 0);
        }
      }
    }
    // ---- normalise, gate, store this lane's row: dims 16 t + 4 q4 + i ----
    if (row_ok) {
      uint16_t* dst = p.out + o_row + l_tok * p.o_sl + h * p.o_sh + gq * p.o_sg;
      const uint16_t* gsrc = p.gate ? p.gate + g_row + l_tok * p.g_sl + h * p.g_sh + gq * p.g_sg + p.g_off : nullptr;
      // every gate piece is loaded before the first store: out may alias gate as far as the compiler knows, so a
      // load after a store waits for it, and the 16 pieces were 16 serial memory round trips at the end of each
      // workgroup
      uint2 gw[D / 16];
      if (gsrc) {
#pragma unroll
        for (int t = 0; t < D / 16; ++t) gw[t] = *reinterpret_cast<const uint2*>(gsrc + 16 * t + 4 * q4);
      }
#pragma unroll
      for (int t = 0; t < D / 16; ++t) {
        const int d = 16 * t + 4 * q4;
        float y[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = l_run > 0.f ? rbf(O[t][i] / l_run) : 0.f;
        if (gsrc) {
          float gt[4];
          unpack2(gw[t].x, gt[0], gt[1]);
          unpack2(gw[t].y, gt[2], gt[3]);
#pragma unroll
          for (int i = 0; i < 4; ++i) y[i] = y[i] * rbf(1.0f / (1.0f + expf(-gt[i])));
        }
        store4_bf16(dst + d, y);
      }
    }
  }

}

// In-place ring write of the tick's valid keys/values, launched after the attention kernel (whose query
// groups of one row run in different workgroups, so none of them may overwrite a column another still reads).
__global__ __launch_bounds__(256) void ring_write_kernel(const RingParams p) {
  const int n = blockIdx.x / p.hkv;
  const int h = blockIdx.x - n * p.hkv;
  // the row's reads are issued together (padded: lens stands in for the offset, unused) and checked without
  // short-circuit branches, each of which made the compiler wait for one read before issuing the next
  const bool padded = p.offsets == nullptr;
  const int64_t slot = p.slots[n];
  int64_t len = p.lens[n];
  const int64_t off = (padded ? p.lens : p.offsets)[n];
  const int64_t start = p.starts[n];
  const bool rejected = (slot < 0) | (slot >= p.ring_rows) | (len < 0) | (len > (padded ? LB_MAX : p.lb));
  if (rejected | (!padded & (len < p.min_len))) return;
  if (padded && len > p.lb) len = p.lb;
  const int64_t base_tok = padded ? 0 : off;
  const int64_t nk_row = padded ? n * p.nk_sn : base_tok * p.nk_sl;
  const int64_t nv_row = padded ? n * p.nv_sn : base_tok * p.nv_sl;
  const int64_t ring_base = ((slot * p.hkv + h) * (int64_t)(p.W + 1)) * D;
  const int c0 = (int)(start % p.W);   // ring column of the tick's first step; j < len <= W follow it
  // 8-byte pieces e = (token j, dims 4 i ..): a thread's pieces are loaded in batches of WB before any of them
  // is stored (the ring and the new rows could alias as far as the compiler knows, so a load after a store
  // would wait for it)
  constexpr int WB = 8;
  const int total = (int)len * (D / 4);
  for (int e0 = threadIdx.x; e0 < total; e0 += 256 * WB) {
    uint2 kw[WB], vw[WB];
#pragma unroll
    for (int u = 0; u < WB; ++u) {
      const int e = min(e0 + 256 * u, total - 1);
      const int j = e / (D / 4);
      const int d = (e - j * (D / 4)) * 4;
      kw[u] = *reinterpret_cast<const uint2*>(p.new_k + nk_row + j * p.nk_sl + h * p.nk_sh + d);
      vw[u] = *reinterpret_cast<const uint2*>(p.new_v + nv_row + j * p.nv_sl + h * p.nv_sh + d);
    }
#pragma unroll
    for (int u = 0; u < WB; ++u) {
      const int e = e0 + 256 * u;
      if (e < total) {
        const int j = e / (D / 4);
        const int d = (e - j * (D / 4)) * 4;
        const int col = c0 + j < p.W ? c0 + j : c0 + j - p.W;
        const int64_t dst = ring_base + (int64_t)col * D + d;
        *reinterpret_cast<uint2*>(p.ring_k + dst) = kw[u];
        *reinterpret_cast<uint2*>(p.ring_v + dst) = vw[u];
      }
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
                                  float scale, int32_t write_ring, int32_t min_len, void* out, int64_t o_sn,
                                  int64_t o_sl, int64_t o_sh, int64_t o_sg, void* stream) {
  using namespace hsg;
  if (n_rows < 0 || lb <= 0 || hkv <= 0 || groups <= 0 || ring_rows <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  if (!q || !ring_k || !ring_v || !new_k || !new_v || !ring_pos || !slots || !starts || !lens || !out)
    return HSG_ERR_ARG;
  if (head_dim != D || window <= 0 || window > W_MAX || window % KB != 0 || lb > LB_MAX) return HSG_ERR_SHAPE;
  if (write_ring && lb > window) return HSG_ERR_SHAPE;  // two steps of one tick would share a ring column
  const int64_t s16[] = {q_sn, q_sl, q_sh, q_sg, nk_sn, nk_sl, nk_sh, nv_sn, nv_sl, nv_sh};
  for (int64_t s : s16)
    if (s % 8) return HSG_ERR_ALIGN;
  const int64_t s4[] = {g_sn, g_sl, g_sh, g_sg, g_off, o_sn, o_sl, o_sh, o_sg};
  for (int64_t s : s4)
    if (s % 4) return HSG_ERR_ALIGN;
  if (!aligned(q, 16) || !aligned(ring_k, 16) || !aligned(ring_v, 16) || !aligned(new_k, 16) ||
      !aligned(new_v, 16) || !aligned(out, 8) || (gate && !aligned(gate, 8)))
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
  p.lb = lb; p.hkv = hkv; p.G = groups; p.scale = scale; p.write_ring = write_ring; p.min_len = min_len;
  p.out = static_cast<uint16_t*>(out); p.o_sn = o_sn; p.o_sl = o_sl; p.o_sh = o_sh; p.o_sg = o_sg;
  p.qgroups = ((groups * lb + 15) / 16 + NW - 1) / NW;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(ring_attn_mfma_kernel, dim3((unsigned)(n_rows * hkv * p.qgroups)), dim3(NW * 64), 0, st, p);
  if (write_ring) hipLaunchKernelGGL(ring_write_kernel, dim3((unsigned)(n_rows * hkv)), dim3(256), 0, st, p);
  return launch_status();
}
