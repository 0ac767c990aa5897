// Chunked gated-delta-rule prefill for gfx950 (WY/UT chunk form on MFMA).
//
// Same recurrence as the slot step (src/hs_guard/engine/fused_kernels.py:166-188), evaluated 64 tokens at a
// time in the chunk form behind FLA's chunk_gated_delta_rule (called at src/hs_guard/runtime.py:80-89 and
// src/hs_guard/engine/bucketed_engine.py:109-111; written out in transformers' torch_chunk_gated_delta_rule):
// per chunk, with G_i the in-chunk cumulative log-decay, raw bf16 rows Kr, Qr, Vr and the per-token l2-norm
// factors rk, rq (rq includes the K^-1/2 scale):
//   A[i,j]  = beta_i rk_i rk_j e^(G_i-G_j) (Kr Kr^T)[i,j]        j < i
//   V'      = (I + A)^-1 (beta . Vr - beta e^G rk . (Kr S))       (forward substitution in 16-token blocks)
//   O       = rq e^G . (Qr S) + P V',   P[i,j] = rq_i rk_j e^(G_i-G_j) (Qr Kr^T)[i,j]   j <= i
//   S       <- e^(G_C) S + Kr^T (rk e^(G_C-G) . V')
// which is the recurrence unrolled over the chunk (v'_t is the rule's beta (v - S^T k) with the decays
// applied in order).
//
// Mapping: one workgroup (4 waves) per (row, value head, 64-column value block); wave w owns value columns
// [16w, 16w+16) of the block and keeps S[:, those columns] (128 x 16 fp32) in MFMA accumulator layout for the
// whole sequence, so the state is read once and written once per call. The accumulator layout of a 16-row
// block (lane l: column l%16, rows 4(l/16)..+3) is exactly the B-operand layout of v_mfma_f32_16x16x16_bf16,
// so S, the substitution's right-hand sides and V' feed the next product from registers; pairs of 16-row
// blocks feed v_mfma_f32_16x16x32_bf16 by ordering its 32 reduction slots as (4 rows of block J, 4 rows of
// block J+1) per lane, with the A operand read in the same order.
// Precision: Kr, Qr, Vr are exact bf16 operands. Every fp32 operand on the state path (S, -A, the diagonal
// inverses, right-hand sides, V', Z) is split into bf16 hi + lo and multiplied in three passes (hi.hi + hi.lo
// + lo.hi, error ~2^-16 relative), so the state keeps fp32-level accuracy; the diagonal 16 x 16 inverses are
// fp32 forward substitution. -A, P and the inverses are written to LDS already split, once per workgroup.
// Two code-generation rules this kernel keeps on gfx950:
//   * one MFMA accumulation chain uses one MFMA shape: a 16x16x16 product accumulating directly onto the
//     result of a 16x16x32 product lost part of that result (found by bisecting a wrong output), so odd
//     blocks are zero-padded 16x16x32 products;
//   * the global prefetch is unconditional (clamped row pointer): a conditional load was compiled as a load
//     through a selected pointer to a stack zero, which forced a full memory wait every chunk.
#include <math.h>

#include "hsg_common.h"

namespace hsg {
namespace {

constexpr int KD = 128;
constexpr int VD = 128;
constexpr int CH = 64;             // tokens per chunk
constexpr int BV = 64;             // value columns per workgroup
constexpr int KS = KD + 8;         // Ks / Qs row stride (bf16): token-major rows of keys
constexpr int TS = CH + 4;         // KTs / VT row stride (bf16): key- / value-major rows of tokens
constexpr int DS = 20;             // diagonal-block row stride (fp32) and diagonal-inverse row stride (bf16)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) short s16x8;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;

struct ChunkParams {
  const uint16_t* qkv;
  int64_t qkv_stride;
  int q_off, k_off, v_off;
  const uint16_t* a;
  const uint16_t* b;
  int64_t ab_stride;
  const uint16_t* A_log;
  const uint16_t* dt_bias;
  void* state;
  int64_t state_rows;
  const int64_t* slots;
  const int64_t* lens;
  const int64_t* offsets;
  int L, H, HV;
  int pairs;                       // n_rows * HV
  float scale;
  uint16_t* o;
  float* sq;
};

__device__ __forceinline__ f32x4 mma16(s16x4 a, s16x4 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ f32x4 mma32(s16x8 a, s16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

__device__ __forceinline__ s16x8 cat(s16x4 x, s16x4 y) { return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7); }

// x = hi + lo with hi = bf16(x) and lo = bf16(x - hi), both round-to-nearest-even. The rounding is done in
// integer arithmetic: a build of this kernel using the compiler's __bf16 conversion produced wrong values in
// a few rows of one tile on gfx950, while the identical kernel with this conversion is exact.
__device__ __forceinline__ void split4(f32x4 x, s16x4& hi, s16x4& lo) {
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint16_t h = f2bf_finite(x[i]);
    hi[i] = (short)h;
    lo[i] = (short)f2bf_finite(x[i] - bf2f(h));
  }
}

__device__ __forceinline__ f32x4 ld4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ s16x4 ld4h(const uint16_t* p) { return *reinterpret_cast<const s16x4*>(p); }

// acc += sum_{J < NJ} M[row block I][col block J] . B_J for a matrix M kept in LDS as bf16 hi / lo planes, read
// at hrow = &Mh[16I + m][4 g], lrow = &Ml[16I + m][4 g] (lane m = l%16, g = l/16); B_J are split bf16 pairs in
// B layout. Three passes per product (hi.hi + hi.lo + lo.hi).
template <int NJ>
__device__ __forceinline__ f32x4 split_product(const uint16_t* hrow, const uint16_t* lrow, const s16x4* bh,
                                               const s16x4* bl, f32x4 acc) {
#pragma unroll
  for (int J = 0; J + 1 < NJ; J += 2) {
    const s16x8 ah = cat(ld4h(hrow + 16 * J), ld4h(hrow + 16 * J + 16));
    const s16x8 al = cat(ld4h(lrow + 16 * J), ld4h(lrow + 16 * J + 16));
    const s16x8 b_h = cat(bh[J], bh[J + 1]), b_l = cat(bl[J], bl[J + 1]);
    acc = mma32(al, b_h, acc);
    acc = mma32(ah, b_l, acc);
    acc = mma32(ah, b_h, acc);
  }
  if constexpr (NJ % 2 == 1) {
    // the odd block rides in a 16x16x32 product with zero upper k-slots: one accumulation chain never mixes
    // MFMA shapes (a 16x16x16 accumulating onto a 16x16x32 result lost that result in some rows)
    constexpr int J = NJ - 1;
    const s16x4 z = {0, 0, 0, 0};
    const s16x8 ah = cat(ld4h(hrow + 16 * J), z), al = cat(ld4h(lrow + 16 * J), z);
    const s16x8 b_h = cat(bh[J], z), b_l = cat(bl[J], z);
    acc = mma32(al, b_h, acc);
    acc = mma32(ah, b_l, acc);
    acc = mma32(ah, b_h, acc);
  }
  return acc;
}

// e^x for x <= 0 on the hardware exp2 (v_exp_f32, 1 ulp): 2^(x log2 e)
__device__ __forceinline__ float exp_nonpos(float x) { return __builtin_amdgcn_exp2f(x * 1.44269504088896341f); }

__device__ __forceinline__ void store_split(uint16_t* hi, uint16_t* lo, float x) {
  const uint16_t h = f2bf_finite(x);
  *hi = h;
  *lo = f2bf_finite(x - bf2f(h));
}

// workgroup barrier that orders LDS only (outstanding global prefetches stay in flight)
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

template <typename ST>
__device__ __forceinline__ float load_state(const ST* p);
template <>
__device__ __forceinline__ float load_state<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_state<uint16_t>(const uint16_t* p) { return h2f(*p); }
__device__ __forceinline__ void store_state(float* p, float x) { *p = x; }
__device__ __forceinline__ void store_state(uint16_t* p, float x) { *p = f2h(x); }

template <typename ST>
__global__ __launch_bounds__(256) void gdn_chunk_kernel(const ChunkParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m16 = lane & 15;
  const int g4 = lane >> 4;
  // the two value blocks of one (row, head) are dispatched 8 workgroups apart, i.e. on the same XCD, so
  // their identical K / Q chunk reads share that XCD's L2
  const int bid = blockIdx.x;
  const int vb = (bid >> 3) & 1;
  const int pair = ((bid >> 4) << 3) | (bid & 7);
  if (pair >= p.pairs) return;
  const int n = pair / p.HV;
  const int hv = pair - n * p.HV;
  const int h = hv / (p.HV / p.H);
  const int64_t slot = p.slots[n];
  int ntok = (int)p.lens[n];
  const bool padded = p.offsets == nullptr;
  if (slot < 0 || slot >= p.state_rows || ntok < 0) ntok = 0;
  if (padded && ntok > p.L) ntok = p.L;
  const int64_t tok0 = padded ? (int64_t)n * p.L : p.offsets[n];
  const int vcol = vb * BV + wave * 16 + m16;          // this lane's value column (accumulator layout)
  const int64_t ostride = (int64_t)p.HV * VD;

  if (padded) {  // positions past the row's length are zeros in the padded layout
    for (int t = ntok + threadIdx.x / BV; t < p.L; t += 256 / BV) {
      const int64_t at = (tok0 + t) * ostride + hv * VD + vb * BV + (threadIdx.x % BV);
      p.o[at] = 0;
      if (p.sq) p.sq[at] = 0.f;
    }
  }
  if (ntok == 0) return;

  __shared__ __align__(16) uint16_t Ks[CH * KS];
  __shared__ __align__(16) uint16_t Qs[CH * KS];
  __shared__ __align__(16) uint16_t KTs[KD * TS];
  __shared__ __align__(16) uint16_t VT[BV * TS];
  // -A (strictly lower) and P (lower incl. diagonal) as bf16 hi / lo planes, token-major rows
  __shared__ __align__(16) uint16_t Ah[CH * TS], Al[CH * TS], Ph[CH * TS], Pl[CH * TS];
  __shared__ __align__(16) float Dg[4 * 16 * DS];                // fp32 diagonal 16 x 16 blocks of A
  __shared__ __align__(16) uint16_t Th[CH * DS], Tl[CH * DS];    // their inverses (rows 16w + i of block w)
  __shared__ __align__(16) float rk_s[CH], rq_s[CH], g_s[CH], b_s[CH], c1_s[CH], d_s[CH], qe_s[CH], G_s[CH], fa_s[CH];
  __shared__ float gc_s;

  // ---- state S[:, vcol] in accumulator layout: block mt holds keys 16 mt + 4 g4 + r ----
  ST* sbase = reinterpret_cast<ST*>(p.state) + ((slot * p.HV + hv) * (int64_t)KD) * VD + vcol;
  f32x4 S[8];
#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) S[mt][r] = load_state<ST>(sbase + (int64_t)(16 * mt + 4 * g4 + r) * VD);

  const float A = expf(bf2f(p.A_log[hv]));
  const float dt = bf2f(p.dt_bias[hv]);

  // ---- staging coordinates: token st_t of the chunk; 16-byte pieces g4 + 4 it ----
  const int st_t = 16 * wave + m16;
  uint4 pk[4], pq[4], pv[2];
  uint16_t pa = 0, pb = 0;   // raw bf16: converting here would make every prefetch wait for its loads
  // Loads are unconditional: a position past the row's end reads the row's first token instead, and its
  // zero beta, rk and rq factors (set at staging) cancel it everywhere, so no select can turn into a
  // memory-backed zero or a branch around the loads.
  auto fetch = [&](int c0) {
    const int64_t tok = tok0 + (c0 + st_t < ntok ? c0 + st_t : 0);
    const uint16_t* row = p.qkv + tok * p.qkv_stride;
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int pc = 8 * (g4 + 4 * it);
      pk[it] = *reinterpret_cast<const uint4*>(row + p.k_off + h * KD + pc);
      pq[it] = *reinterpret_cast<const uint4*>(row + p.q_off + h * KD + pc);
    }
#pragma unroll
    for (int it = 0; it < 2; ++it) {
      const int pc = 8 * (g4 + 4 * it);
      pv[it] = *reinterpret_cast<const uint4*>(row + p.v_off + hv * VD + vb * BV + pc);
    }
    pa = p.a[tok * p.ab_stride + hv];
    pb = p.b[tok * p.ab_stride + hv];
  };

  fetch(0);
  for (int c0 = 0; c0 < ntok; c0 += CH) {
    const int nv = min(CH, ntok - c0);
    lds_barrier();  // every read of the previous chunk's LDS data is done
    {
      float kk = 0.f, qq = 0.f;
#pragma unroll
      for (int it = 0; it < 4; ++it) {
        const int pc = 8 * (g4 + 4 * it);
        *reinterpret_cast<uint4*>(&Ks[st_t * KS + pc]) = pk[it];
        *reinterpret_cast<uint4*>(&Qs[st_t * KS + pc]) = pq[it];
        const uint32_t kw[4] = {pk[it].x, pk[it].y, pk[it].z, pk[it].w};
        const uint32_t qw[4] = {pq[it].x, pq[it].y, pq[it].z, pq[it].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          KTs[(pc + 2 * e) * TS + st_t] = (uint16_t)(kw[e] & 0xffffu);
          KTs[(pc + 2 * e + 1) * TS + st_t] = (uint16_t)(kw[e] >> 16);
          float x0, x1, y0, y1;
          unpack2(kw[e], x0, x1);
          unpack2(qw[e], y0, y1);
          kk += x0 * x0 + x1 * x1;
          qq += y0 * y0 + y1 * y1;
        }
      }
#pragma unroll
      for (int it = 0; it < 2; ++it) {
        const int pc = 8 * (g4 + 4 * it);
        const uint32_t vw[4] = {pv[it].x, pv[it].y, pv[it].z, pv[it].w};
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          VT[(pc + 2 * e) * TS + st_t] = (uint16_t)(vw[e] & 0xffffu);
          VT[(pc + 2 * e + 1) * TS + st_t] = (uint16_t)(vw[e] >> 16);
        }
      }
      kk = xor_add<16>(kk);
      kk = xor_add<32>(kk);
      qq = xor_add<16>(qq);
      qq = xor_add<32>(qq);
      if (g4 == 0) {
        const bool ok = st_t < nv;
        rk_s[st_t] = ok ? 1.0f / sqrtf(kk + 1e-6f) : 0.f;
        rq_s[st_t] = ok ? p.scale / sqrtf(qq + 1e-6f) : 0.f;
        const float x = bf2f(pa) + dt;
        g_s[st_t] = ok ? -A * (x > 20.0f ? x : logf(1.0f + expf(x))) : 0.f;
        b_s[st_t] = ok ? sigmoidf_(bf2f(pb)) : 0.f;
      }
    }
    if (c0 + CH < ntok) fetch(c0 + CH);  // next chunk's loads stay in flight during this chunk's math
    lds_barrier();

    // ---- in-chunk cumulative decay and per-token factors (wave 0) ----
    if (wave == 0) {
      float x = g_s[lane];
#pragma unroll
      for (int d = 1; d < 64; d <<= 1) {
        const float y = __shfl_up(x, d, 64);
        if (lane >= d) x += y;
      }
      const float GC = __shfl(x, 63, 64);
      const float eg = exp_nonpos(x);
      G_s[lane] = x;
      c1_s[lane] = b_s[lane] * eg * rk_s[lane];
      fa_s[lane] = b_s[lane] * rk_s[lane];
      d_s[lane] = rk_s[lane] * exp_nonpos(GC - x);
      qe_s[lane] = rq_s[lane] * eg;
      if (lane == 0) gc_s = exp_nonpos(GC);
    }

    // ---- Kr Kr^T and Qr Kr^T on the 10 lower 16 x 16 tiles each; tile u of wave w is number w + 4u ----
    f32x4 gt[5];
#pragma unroll
    for (int u = 0; u < 5; ++u) {
      const int tau = wave + 4 * u;
      const bool qk = tau >= 10;
      const int idx = qk ? tau - 10 : tau;
      const int I = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
      const int J = idx - I * (I + 1) / 2;
      const uint16_t* arow = (qk ? Qs : Ks) + (16 * I + m16) * KS + 8 * g4;
      const uint16_t* brow = Ks + (16 * J + m16) * KS + 8 * g4;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int ks = 0; ks < 4; ++ks)
        acc = mma32(*reinterpret_cast<const s16x8*>(arow + 32 * ks), *reinterpret_cast<const s16x8*>(brow + 32 * ks),
                    acc);
      gt[u] = acc;
    }

    // ---- Y = Kr S and QS = Qr S for this wave's 16 columns (S split hi / lo, key blocks paired) ----
    s16x4 Sh[8], Sl[8];
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) split4(S[mt], Sh[mt], Sl[mt]);
    f32x4 Y[4], QS[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 y = {0.f, 0.f, 0.f, 0.f}, qs = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = Ks + (16 * I + m16) * KS + 4 * g4;
      const uint16_t* qrow = Qs + (16 * I + m16) * KS + 4 * g4;
#pragma unroll
      for (int q2 = 0; q2 < 4; ++q2) {
        const s16x8 ka = cat(ld4h(krow + 32 * q2), ld4h(krow + 32 * q2 + 16));
        const s16x8 qa = cat(ld4h(qrow + 32 * q2), ld4h(qrow + 32 * q2 + 16));
        const s16x8 sh = cat(Sh[2 * q2], Sh[2 * q2 + 1]), sl = cat(Sl[2 * q2], Sl[2 * q2 + 1]);
        y = mma32(ka, sl, y);
        y = mma32(ka, sh, y);
        qs = mma32(qa, sl, qs);
        qs = mma32(qa, sh, qs);
      }
      Y[I] = y;
      QS[I] = qs;
    }
    lds_barrier();  // per-token factors are in LDS

    // ---- scale the Gram tiles into -A and P. Only P's diagonal tiles need the causal mask: the substitution
    // reads A's off-diagonal tiles only and the diagonal inverses read below the diagonal only. ----
    {
      f32x4 fr[5], Gr[5];
      float rkc[5], Gc[5];
#pragma unroll
      for (int u = 0; u < 5; ++u) {
        const int tau = wave + 4 * u;
        const bool qk = tau >= 10;
        const int idx = qk ? tau - 10 : tau;
        const int I = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
        const int J = idx - I * (I + 1) / 2;
        const int i0 = 16 * I + 4 * g4;
        fr[u] = ld4f(qk ? &rq_s[i0] : &fa_s[i0]);
        Gr[u] = ld4f(&G_s[i0]);
        rkc[u] = rk_s[16 * J + m16];
        Gc[u] = G_s[16 * J + m16];
      }
#pragma unroll
      for (int u = 0; u < 5; ++u) {
        const int tau = wave + 4 * u;
        const bool qk = tau >= 10;
        const int idx = qk ? tau - 10 : tau;
        const int I = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
        const int J = idx - I * (I + 1) / 2;
        const int i0 = 16 * I + 4 * g4;
        const int j = 16 * J + m16;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const float v = fr[u][r] * rkc[u] * exp_nonpos(fminf(Gr[u][r] - Gc[u], 0.f)) * gt[u][r];
          if (!qk) {
            store_split(&Ah[(i0 + r) * TS + j], &Al[(i0 + r) * TS + j], -v);
            if (I == J) Dg[(i0 + r) * DS + m16] = -v;
          } else {
            // keep = 1 when row >= column inside a diagonal tile (sign bit of column - row - 1)
            const float keep = I == J ? (float)((uint32_t)(m16 - (4 * g4 + r) - 1) >> 31) : 1.f;
            store_split(&Ph[(i0 + r) * TS + j], &Pl[(i0 + r) * TS + j], v * keep);
          }
        }
      }
    }
    // ---- right-hand sides R = beta . V - beta e^G rk . Y (in place in Y) ----
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int i0 = 16 * I + 4 * g4;
      const f32x4 bt = ld4f(&b_s[i0]), c1 = ld4f(&c1_s[i0]);
      float v4[4];
      load4_bf16(&VT[(wave * 16 + m16) * TS + i0], v4);
#pragma unroll
      for (int r = 0; r < 4; ++r) Y[I][r] = bt[r] * v4[r] - c1[r] * Y[I][r];
    }
    lds_barrier();  // A and P are complete

    // ---- wave w inverts diagonal block w of (I + A) by fp32 forward substitution (lane m16 = column) ----
    {
      const float* nb = Dg + (16 * wave) * DS;   // -A of the block
      float t[16];
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        float s0 = (i == m16) ? 1.f : 0.f, s1 = 0.f, s2 = 0.f, s3 = 0.f;
#pragma unroll
        for (int k = 0; k < i; ++k) {
          const float a = nb[i * DS + k];
          if ((k & 3) == 0) s0 += a * t[k];
          else if ((k & 3) == 1) s1 += a * t[k];
          else if ((k & 3) == 2) s2 += a * t[k];
          else s3 += a * t[k];
        }
        t[i] = (s0 + s1) + (s2 + s3);
      }
      // every lane group computed the same column; group g4 writes rows 4 g4 .. 4 g4 + 3 of it
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float ti = g4 == 0 ? t[i] : g4 == 1 ? t[4 + i] : g4 == 2 ? t[8 + i] : t[12 + i];
        store_split(&Th[(wave * 16 + 4 * g4 + i) * DS + m16], &Tl[(wave * 16 + 4 * g4 + i) * DS + m16], ti);
      }
    }
    lds_barrier();  // diagonal inverses are complete

    // ---- V'_I = T_II (R_I - sum_{J<I} A_IJ V'_J), all in this wave's registers ----
    s16x4 Vh[4], Vl[4];
    f32x4 Vp[4];
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const int arow = (16 * I + m16) * TS + 4 * g4;
      if (I == 1) acc = split_product<1>(Ah + arow, Al + arow, Vh, Vl, acc);
      if (I == 2) acc = split_product<2>(Ah + arow, Al + arow, Vh, Vl, acc);
      if (I == 3) acc = split_product<3>(Ah + arow, Al + arow, Vh, Vl, acc);
      const f32x4 x = Y[I] + acc;
      s16x4 xh, xl;
      split4(x, xh, xl);
      const s16x4 th = ld4h(&Th[(I * 16 + m16) * DS + 4 * g4]), tl = ld4h(&Tl[(I * 16 + m16) * DS + 4 * g4]);
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
      v = mma16(tl, xh, v);
      v = mma16(th, xl, v);
      v = mma16(th, xh, v);
      Vp[I] = v;
      split4(v, Vh[I], Vl[I]);
    }

    // ---- O = rq e^G . QS + P V' ----
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      const int i0 = 16 * I + 4 * g4;
      const f32x4 qe = ld4f(&qe_s[i0]);
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const int prow = (16 * I + m16) * TS + 4 * g4;
      if (I == 0) acc = split_product<1>(Ph + prow, Pl + prow, Vh, Vl, acc);
      if (I == 1) acc = split_product<2>(Ph + prow, Pl + prow, Vh, Vl, acc);
      if (I == 2) acc = split_product<3>(Ph + prow, Pl + prow, Vh, Vl, acc);
      if (I == 3) acc = split_product<4>(Ph + prow, Pl + prow, Vh, Vl, acc);
      const f32x4 o = QS[I] * qe + acc;
      uint16_t* orow = p.o + (tok0 + c0 + i0) * ostride + hv * VD + vcol;
      if (nv == CH && !p.sq) {   // whole chunk, no sq: no per-element predicates
#pragma unroll
        for (int r = 0; r < 4; ++r) orow[r * ostride] = f2bf_finite(o[r]);
      } else {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if (i0 + r < nv) {
            const uint16_t ob = f2bf_finite(o[r]);
            orow[r * ostride] = ob;
            if (p.sq) {
              const float x = bf2f(ob);
              p.sq[(tok0 + c0 + i0 + r) * ostride + hv * VD + vcol] = x * x;
            }
          }
        }
      }
    }

    // ---- S <- e^(G_C) S + Kr^T Z,  Z = rk e^(G_C - G) . V' (token blocks paired) ----
    s16x4 Zh[4], Zl[4];
#pragma unroll
    for (int J = 0; J < 4; ++J) {
      const f32x4 d = ld4f(&d_s[16 * J + 4 * g4]);
      split4(Vp[J] * d, Zh[J], Zl[J]);
    }
    const float gc = gc_s;
#pragma unroll
    for (int mt = 0; mt < 8; ++mt) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      const uint16_t* krow = KTs + (16 * mt + m16) * TS + 4 * g4;
#pragma unroll
      for (int J = 0; J < 4; J += 2) {
        const s16x8 ka = cat(ld4h(krow + 16 * J), ld4h(krow + 16 * J + 16));
        acc = mma32(ka, cat(Zl[J], Zl[J + 1]), acc);
        acc = mma32(ka, cat(Zh[J], Zh[J + 1]), acc);
      }
      S[mt] = S[mt] * gc + acc;
    }
  }

#pragma unroll
  for (int mt = 0; mt < 8; ++mt)
#pragma unroll
    for (int r = 0; r < 4; ++r) store_state(sbase + (int64_t)(16 * mt + 4 * g4 + r) * VD, S[mt][r]);
}

}  // namespace
}  // namespace hsg

using hsg::ChunkParams;

extern "C" int hsg_gdn_chunk_prefill(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off,
                                     int32_t v_off, const void* a, const void* b, int64_t ab_stride,
                                     const void* A_log, const void* dt_bias, void* state, int32_t state_dtype,
                                     int64_t state_rows, const int64_t* slots, const int64_t* lens,
                                     const int64_t* offsets, int32_t n_rows, int32_t L, int32_t H, int32_t HV,
                                     int32_t K, int32_t V, float scale, void* o, float* sq, void* stream) {
  ChunkParams p;
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qkv_stride = qkv_stride;
  p.q_off = q_off;
  p.k_off = k_off;
  p.v_off = v_off;
  p.a = static_cast<const uint16_t*>(a);
  p.b = static_cast<const uint16_t*>(b);
  p.ab_stride = ab_stride;
  p.A_log = static_cast<const uint16_t*>(A_log);
  p.dt_bias = static_cast<const uint16_t*>(dt_bias);
  p.state = state;
  p.state_rows = state_rows;
  p.slots = slots;
  p.lens = lens;
  p.offsets = offsets;
  p.L = L;
  p.H = H;
  p.HV = HV;
  p.scale = scale;
  p.o = static_cast<uint16_t*>(o);
  p.sq = sq;
  if (n_rows < 0 || H <= 0 || HV <= 0 || L < 0 || state_rows <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  if (!qkv || !a || !b || !A_log || !dt_bias || !state || !slots || !lens || !o) return HSG_ERR_ARG;
  if (offsets == nullptr && L <= 0) return HSG_ERR_ARG;
  if (K != hsg::KD || V != hsg::VD || HV % H != 0) return HSG_ERR_SHAPE;
  if (state_dtype != HSG_STATE_F32 && state_dtype != HSG_STATE_F16) return HSG_ERR_ARG;
  if (!hsg::aligned(qkv, 16) || qkv_stride % 8 || q_off % 8 || k_off % 8 || v_off % 8) return HSG_ERR_ALIGN;
  if (!hsg::aligned(state, 16) || !hsg::aligned(o, 2) || (sq && !hsg::aligned(sq, 4))) return HSG_ERR_ALIGN;
  if ((int64_t)n_rows * HV > (int64_t)1 << 26) return HSG_ERR_SHAPE;
  p.pairs = n_rows * HV;
  const dim3 grid((unsigned)(((p.pairs + 7) / 8) * 16));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (state_dtype == HSG_STATE_F32)
    hipLaunchKernelGGL((hsg::gdn_chunk_kernel<float>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((hsg::gdn_chunk_kernel<uint16_t>), grid, dim3(256), 0, s, p);
  return hsg::launch_status();
}
