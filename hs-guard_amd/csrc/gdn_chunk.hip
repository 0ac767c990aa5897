// Chunked gated-delta-rule prefill for gfx950 (WY/UT chunk form on MFMA), as two kernels.
//
// Same recurrence as the slot step (src/hs_guard/engine/fused_kernels.py:166-188), evaluated 64 tokens at a
// time in the chunk form behind FLA's chunk_gated_delta_rule (called at src/hs_guard/runtime.py:80-89 and
// src/hs_guard/engine/bucketed_engine.py:109-111; written out in transformers' torch_chunk_gated_delta_rule):
// per chunk, with G_i the in-chunk cumulative log-decay, raw bf16 rows Kr, Qr, Vr and the per-token l2-norm
// factors rk, rq (rq includes the K^-1/2 scale):
//   A[i,j]  = beta_i rk_i rk_j e^(G_i-G_j) (Kr Kr^T)[i,j]        j < i
//   M'      = (I + A)^-1 diag(beta)
//   V'      = M' (Vr - e^G rk . (Kr S))                          (= (I + A)^-1 (beta Vr - beta e^G rk Kr S))
//   O       = rq e^G . (Qr S) + P V',   P[i,j] = rq_i rk_j e^(G_i-G_j) (Qr Kr^T)[i,j]   j <= i
//   S       <- e^(G_C) S + Kr^T (rk e^(G_C-G) . V')
// which is the recurrence unrolled over the chunk (v'_t is the rule's beta (v - S^T k) with the decays
// applied in order).
//
// Only the last three lines involve the state. gdn_chunk_prep_kernel computes everything else for every
// (row, chunk, value head) at once, in parallel: M' and P as scaled fp16 hi / lo planes and the per-token factors
// e^G rk, rq e^G, rk e^(G_C-G) and e^(G_C), into a workspace. gdn_chunk_state_kernel then walks each row's
// chunks in order with only the state products on its chain: per chunk Y = Kr S and Qr S, Z = Vr - e^G rk . Y,
// V' = M' Z (no substitution chain: M' is explicit), O, and the state update.
//
// Prep mapping: one workgroup (4 waves) per (row, chunk, value head). Kr Kr^T and Qr Kr^T on 16 x 16 tiles,
// scaled into -A (LDS) and P (workspace); the four diagonal 16 x 16 blocks of I + A are inverted by fp32
// forward substitution; wave w then solves (I + A) M[:, 16w..16w+16) = I[:, 16w..] block by block, so the
// inverse is explicit, and scales its columns by beta.
// State mapping: one workgroup (8 waves) per (row, value head, 64-column value block), rows with the most
// chunks dispatched first (gdn_chunk_order_kernel). Chain wave w (0-3) owns value columns [16w, 16w+16) of the
// block and keeps S[:, those columns] (128 x 16 fp32) in MFMA accumulator layout for the whole sequence, so the
// state is read once and written once per call; output wave 4 + w computes Q S and O for the same columns from
// the split S and V' the chain wave hands over through LDS. The accumulator layout of a 16-row block (lane l:
// column l%16, rows 4(l/16)..+3) is exactly the B-operand layout of a 16x16x16 MFMA, so S, Z and V'
// feed the next product from registers; pairs of 16-row blocks feed v_mfma_f32_16x16x32_f16 by ordering its
// 32 reduction slots as (4 rows of block J, 4 rows of block J+1) per lane, with the A operand read in the same
// order.
// Precision: Kr, Qr, Vr are exact bf16 values (and exact in fp16, which holds bf16's 8-bit significands). The
// prep kernel forms M' in fp32 throughout (fp32 MFMA for the block substitution). On the state path every fp32
// operand (S, Z, V', W, and the M', P planes) is scaled by a power of two that puts its largest magnitude just
// below 2^14 (S, Z, V', W: per value column, the direction every product using them reduces along), then split into fp16 hi + fp16 lo of the remainder (x 2^s = hi + lo + O(2^-22 |x 2^s|)), and
// multiplied in three fp16 MFMA passes (lo.hi + hi.lo + hi.hi), or two when the other operand is an exact
// input row; the accumulator is scaled back by 2^-s (exact). That keeps every product within ~2^-22 of fp32
// (a bf16 hi + lo split reaches only ~2^-17, which moved one bf16 output in 300 instead of one in 10,000).
// Two code-generation rules these kernels keep on gfx950:
//   * one MFMA accumulation chain uses one MFMA shape: a 16x16x16 product accumulating directly onto the
//     result of a 16x16x32 product lost part of that result (found by bisecting a wrong output), so odd
//     blocks are zero-padded 16x16x32 products;
//   * the global prefetch is unconditional (clamped row pointer): a conditional load was compiled as a load
//     through a selected pointer to a stack zero, which forced a full memory wait every chunk;
//   * every value one lane stores to LDS and another lane of the same wave reads passes a fenced barrier in
//     between: the compiler orders LDS accesses per lane only, and moved a read above another lane's store.
#include <math.h>

#include "hsg_common.h"

namespace hsg {
namespace {

constexpr int KD = 128;
constexpr int VD = 128;
constexpr int CH = 64;             // tokens per chunk
constexpr int BV = 64;             // value columns per workgroup
constexpr int KS = KD + 8;         // Ks / Qs row stride (bf16): token-major rows of keys
constexpr int AS = CH + 4;         // row stride (fp32) of the prep kernel's -A in LDS: a row read of 16 lanes x
                                   // 4 k-slots hits 64 distinct banks
constexpr int VS = BV + 16;        // Vs row stride (bf16): 40 dwords, so the 4 x 4 pieces of a transpose read
                                   // fall in 16 distinct bank pairs
constexpr int DS = 20;             // diagonal-block row stride (fp32) and diagonal-inverse row stride (bf16)
constexpr int PW = CH;             // row width (bf16) of the workspace planes M', P (swizzled rows, see swz)
constexpr int PL = CH * PW;        // one 64 x 64 bf16 plane of the workspace (also the state kernel's LDS layout)
constexpr int VEC = 256;           // per-token factor floats of a workspace unit: e^G rk, rq e^G, rk e^(G_C-G),
                                   // then e^(G_C), the inverse scale of the M' planes and padding
// one workspace unit per (row, chunk, value head): planes M'hi, M'lo, Phi, Plo, then the factors
constexpr int UNIT_BYTES = 4 * PL * 2 + VEC * 4;
constexpr int ORDER_MAX = 4096;    // rows ranked by the order kernel (more rows keep their given order)

typedef __attribute__((ext_vector_type(8))) __bf16 bf16x8;
typedef __attribute__((ext_vector_type(8))) _Float16 f16x8;
typedef __attribute__((ext_vector_type(4))) _Float16 f16x4;
typedef __attribute__((ext_vector_type(8))) short s16x8;
typedef __attribute__((ext_vector_type(4))) short s16x4;
typedef __attribute__((ext_vector_type(4))) float f32x4;
typedef __attribute__((ext_vector_type(8))) float f32x8;

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
  int max_chunks;                  // ceil(L / CH): workspace units per (row, value head)
  int min_len;                     // rows with fewer tokens are left alone
  float scale;
  uint16_t* o;
  float* sq;
  uint8_t* ws;
  int32_t* order;                  // state kernel row order (in the workspace after the units)
  // gated epilogue (hsg_gdn_chunk_prefill_gated): out = gated RMSNorm of o with z
  const uint16_t* z;
  int64_t z_stride;
  const uint16_t* norm_w;
  float eps;
  uint16_t* out;
};

// bf16 operands (the prep kernel's Gram tiles of the raw rows)
__device__ __forceinline__ f32x4 mma32(s16x8 a, s16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b),
                                                 c, 0, 0, 0);
}

// fp16 operands (the state kernel's products)
__device__ __forceinline__ f32x4 mmh32(s16x8 a, s16x8 b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0, 0,
                                                0);
}

// fp32 operands, one k-slot per lane group (the prep kernel's block substitution): lane l supplies A[l % 16][l / 16]
// and B[l / 16][l % 16] of a 16 x 4 by 4 x 16 product
__device__ __forceinline__ f32x4 mmf4(float a, float b, f32x4 c) {
  return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// 2^e as a float and its inverse, e chosen so that amax * 2^e lies in [2^13, 2^14): the scaled values stay well inside
// fp16's range (65504) and the fp16 remainders of all values down to ~2^-17 of the largest stay normal. amax 0, NaN
// or infinite: scale 1. e is clamped to [-100, 100].
__device__ __forceinline__ float pow2_scale(float amax, float* inv) {
  int e = 0;
  if (amax > 0.f && amax < INFINITY) e = 140 - (int)((__float_as_uint(amax) >> 23) & 0xffu);
  e = e < -100 ? -100 : (e > 100 ? 100 : e);
  *inv = __uint_as_float((uint32_t)(127 - e) << 23);
  return __uint_as_float((uint32_t)(127 + e) << 23);
}

// y = x * scale (scale a power of two) as fp16 hi + fp16 lo of the remainder: y = hi + lo + O(2^-22 |y|)
__device__ __forceinline__ void split4h(f32x4 x, float scale, s16x4& hi, s16x4& lo) {
  const f32x4 y = x * scale;
  const f16x4 h = __builtin_convertvector(y, f16x4);
  const f16x4 l = __builtin_convertvector(y - __builtin_convertvector(h, f32x4), f16x4);
  hi = __builtin_bit_cast(s16x4, h);
  lo = __builtin_bit_cast(s16x4, l);
}

// largest value over the four lanes of one accumulator column (lanes l, l ^ 16, l ^ 32, l ^ 48): the scale of a
// split operand is shared by the values of one column, which is all that a product reducing along the column
// (over keys or over tokens) needs
__device__ __forceinline__ float col_max(float x) { return max_pair32(max_pair16(x)); }

__device__ __forceinline__ float absmax4(f32x4 x, float m) {
  return fmaxf(fmaxf(m, fmaxf(fabsf(x[0]), fabsf(x[1]))), fmaxf(fabsf(x[2]), fabsf(x[3])));
}

// 8 raw bf16 values (one 16-byte piece of a K or Q row) as 8 fp16 values: exact, fp16 holds bf16's significands
// (magnitudes below 2^-14 become fp16 subnormals; their products are below fp32 resolution of the sums they join)
__device__ __forceinline__ u32x4 bf16x8_to_f16x8(u32x4 w) {
  f32x8 f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    f[2 * i] = __uint_as_float(w[i] << 16);
    f[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
  }
  return __builtin_bit_cast(u32x4, __builtin_convertvector(f, f16x8));
}

__device__ __forceinline__ s16x8 cat(s16x4 x, s16x4 y) { return __builtin_shufflevector(x, y, 0, 1, 2, 3, 4, 5, 6, 7); }

__device__ __forceinline__ f32x4 ld4f(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ s16x4 ld4h(const uint16_t* p) { return *reinterpret_cast<const s16x4*>(p); }

// e^x for x <= 0 given in fp64, on the hardware exp2 (v_exp_f32, 1 ulp): x log2 e = n + f is split in fp64 (n
// integer, 0 <= f < 1) and e^x = 2^f 2^n, so the fp32 rounding of the argument costs ~2^-25 relative whatever |x|
// is (rounding x log2 e itself to fp32 costs ~|x| 2^-24, 3e-6 at |x| = 50)
__device__ __forceinline__ float exp_nonpos_d(double x) {
  const double y = x * 1.4426950408889634;
  const double n = floor(y);
  return ldexpf(__builtin_amdgcn_exp2f((float)(y - n)), (int)n);
}


// LDS transpose read (ds_read_b64_tr_b16): within each group of 16 lanes, lane 4q + e receives element e of
// the 4-element (8-byte) vectors addressed by lanes q, q + 4, q + 8, q + 12 of its group. With a row-major
// tile, lane s of a group addressing row r0 + (s >> 2), columns c0 + 4 (s & 3) .. +3 therefore receives
// column c0 + s of rows r0 .. r0 + 3: the MFMA operand layout of the transposed tile.
__device__ __forceinline__ s16x4 ld4h_tr(const uint16_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((__attribute__((address_space(3))) s16x4*)(p));
}

// The state kernel's K and Q tiles are unpadded 256-byte token rows whose 8-byte pieces are permuted within each
// row: logical piece c of row r is stored at piece c ^ swz(r). A row read (16 lanes: 16 consecutive rows, one
// piece) and a transpose read (16 lanes: 4 rows x 4 consecutive pieces) then both touch 16 distinct 8-byte bank
// pairs, where any padding of the row leaves one of the two patterns with 2- to 4-way bank conflicts.
__device__ __forceinline__ int swz(int r) { return ((r & 3) << 2) | ((r >> 2) & 3); }

// offset (bf16) of logical 4-element piece c in swizzled row r
__device__ __forceinline__ int swz_at(int r, int c) { return r * KD + 4 * (c ^ swz(r)); }

// the same for the 64-column planes M' and P (16 pieces per row; the XOR permutes all of them)
__device__ __forceinline__ int pw_at(int r, int c) { return r * PW + 4 * (c ^ swz(r)); }

// The lower-triangle blocks of a plane pair (hi then lo plane) are the only part of M' and P the state kernel
// reads: 320 16-byte slots per plane, row block I holding 2 (I + 1) slots per row. Slot q of the pair holds 16-byte
// piece k of its row's lower triangle, i.e. logical pieces 4 (k / 2) .. +3, whose physical 16-byte slot is
// 2 ((k / 2) ^ (swz(row) >> 2)) + k % 2 (the XOR keeps aligned groups of four). Returns its offset (bf16) in
// the pair.
constexpr int TRI_SLOTS = 320;
__device__ __forceinline__ int tri_slot_offset(int q) {
  const int e = q >= TRI_SLOTS;
  const int qq = q - TRI_SLOTS * e;
  const int I = qq >= 192 ? 3 : qq >= 96 ? 2 : qq >= 32 ? 1 : 0;
  const int n2 = 2 * (I + 1);
  const int q2 = qq - (I == 3 ? 192 : I == 2 ? 96 : I == 1 ? 32 : 0);
  const int row = 16 * I + q2 / n2;
  const int k = q2 - (q2 / n2) * n2;
  return e * PL + row * PW + 8 * (2 * ((k >> 1) ^ (swz(row) >> 2)) + (k & 1));
}

// acc += sum_{J < NJ} M[row block I][col block J] . B_J for a matrix M kept in LDS as scaled fp16 hi / lo planes
// (swizzled rows): hrow / lrow = row 16 I + m of the hi / lo planes, po[J] = offset of the lane's logical piece
// 4 J + g in that row (rows 16 I + m share swz(m)); B_J are scaled fp16 hi / lo pairs in B layout. Three passes per
// product (lo.hi + hi.lo + hi.hi). TR: the same operands with the MFMA operand order swapped, which yields the
// transposed product (sum_J B_J^T M_IJ^T) in accumulator layout. The odd block rides in a 16x16x32 product with
// zero upper k-slots: one accumulation chain never mixes MFMA shapes (a 16x16x16 accumulating onto a 16x16x32
// result lost that result in some rows).
template <int NJ, bool TR = false>
__device__ __forceinline__ f32x4 split_product_sw(const uint16_t* hrow, const uint16_t* lrow, const int* po,
                                                  const s16x4* bh, const s16x4* bl, f32x4 acc) {
  auto mm = [](s16x8 m, s16x8 b, f32x4 c) { return TR ? mmh32(b, m, c) : mmh32(m, b, c); };
#pragma unroll
  for (int J = 0; J + 1 < NJ; J += 2) {
    const s16x8 ah = cat(ld4h(hrow + po[J]), ld4h(hrow + po[J + 1]));
    const s16x8 al = cat(ld4h(lrow + po[J]), ld4h(lrow + po[J + 1]));
    const s16x8 b_h = cat(bh[J], bh[J + 1]), b_l = cat(bl[J], bl[J + 1]);
    acc = mm(al, b_h, acc);
    acc = mm(ah, b_l, acc);
    acc = mm(ah, b_h, acc);
  }
  if constexpr (NJ % 2 == 1) {
    constexpr int J = NJ - 1;
    const s16x4 z = {0, 0, 0, 0};
    const s16x8 ah = cat(ld4h(hrow + po[J]), z), al = cat(ld4h(lrow + po[J]), z);
    const s16x8 b_h = cat(bh[J], z), b_l = cat(bl[J], z);
    acc = mm(al, b_h, acc);
    acc = mm(ah, b_l, acc);
    acc = mm(ah, b_h, acc);
  }
  return acc;
}

template <typename ST>
__device__ __forceinline__ float load_state(const ST* p);
template <>
__device__ __forceinline__ float load_state<float>(const float* p) { return *p; }
template <>
__device__ __forceinline__ float load_state<uint16_t>(const uint16_t* p) { return h2f(*p); }
__device__ __forceinline__ void store_state(float* p, float x) { *p = x; }
__device__ __forceinline__ void store_state(uint16_t* p, float x) { *p = f2h(x); }

// Tokens of row n (0 for a slot outside the pool or a rejected row) and the row's first token.
// Padded layout: at most L tokens; packed layout: rows longer than L are rejected (L sizes the workspace).
__device__ __forceinline__ int row_tokens(const ChunkParams& p, int n, int64_t& slot, int64_t& tok0) {
  slot = p.slots[n];
  const int64_t len = p.lens[n];
  const bool padded = p.offsets == nullptr;
  tok0 = padded ? (int64_t)n * p.L : p.offsets[n];
  if (slot < 0 || slot >= p.state_rows || len <= 0 || len < p.min_len) return 0;
  if (padded) return (int)min(len, (int64_t)p.L);
  return len > p.L ? 0 : (int)len;
}

__device__ __forceinline__ uint8_t* unit_ptr(const ChunkParams& p, int n, int c, int hv) {
  return p.ws + (((int64_t)n * p.max_chunks + c) * p.HV + hv) * (int64_t)UNIT_BYTES;
}

// ---------------------------------------------------------------------------------------------------------
// Prep: M' = (I + A)^-1 diag(beta), P and the per-token factors of one (row, chunk, value head).
// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(256) void gdn_chunk_prep_kernel(const ChunkParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int m16 = lane & 15;
  const int g4 = lane >> 4;
  const int bid = blockIdx.x;
  const int hv = bid % p.HV;
  const int nc = bid / p.HV;
  const int c = nc % p.max_chunks;
  const int n = nc / p.max_chunks;
  int64_t slot, tok0;
  const int ntok = row_tokens(p, n, slot, tok0);
  const int c0 = c * CH;
  if (c0 >= ntok) return;
  const int nv = min(CH, ntok - c0);
  const int h = hv / (p.HV / p.H);
  uint8_t* unit = unit_ptr(p, n, c, hv);
  uint16_t* Mh_g = reinterpret_cast<uint16_t*>(unit);   // M'hi, then M'lo at + PL
  uint16_t* Ph_g = Mh_g + 2 * PL;
  uint16_t* Pl_g = Mh_g + 3 * PL;
  float* vec_g = reinterpret_cast<float*>(unit + 4 * PL * 2);

  // Once the Gram tiles are done (a barrier apart) Qs holds -A in fp32 and Ks the substitution's M blocks in fp32,
  // then the M' output planes
  __shared__ __align__(16) uint16_t Ks[CH * KS];
  __shared__ __align__(16) uint16_t Qs[CH * KS];
  float* const nA = reinterpret_cast<float*>(Qs);                // -A (strictly lower), fp32, row stride AS
  __shared__ __align__(16) float Dg[4 * 16 * DS];                // fp32 diagonal 16 x 16 blocks of -A
  __shared__ __align__(16) float Tf[CH * DS];                    // their inverses, fp32 (rows 16w + i of block w)
  __shared__ __align__(16) float rk_s[CH], rq_s[CH], g_s[CH], b_s[CH], fa_s[CH];
  __shared__ __align__(16) double G_s[CH];   // in-chunk cumulative log-decay (see the scan below)
  __shared__ float red_s[4];

  // ---- stage token st_t: raw K, Q rows into LDS, l2-norm factors, gates. Past the row's end the chunk's
  // first token is read instead and its zero beta, rk and rq cancel it everywhere. ----
  const int st_t = 16 * wave + m16;
  const uint16_t A_raw = p.A_log[hv], dt_raw = p.dt_bias[hv];   // issued with the token loads
  {
    const int64_t tok = tok0 + c0 + (st_t < nv ? st_t : 0);
    const uint16_t* row = p.qkv + tok * p.qkv_stride;
    uint4 pk[4], pq[4];
#pragma unroll
    for (int it = 0; it < 4; ++it) {
      const int pc = 8 * (g4 + 4 * it);
      pk[it] = *reinterpret_cast<const uint4*>(row + p.k_off + h * KD + pc);
      pq[it] = *reinterpret_cast<const uint4*>(row + p.q_off + h * KD + pc);
    }
    const uint16_t pa = p.a[tok * p.ab_stride + hv];
    const uint16_t pb = p.b[tok * p.ab_stride + hv];
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
        float x0, x1, y0, y1;
        unpack2(kw[e], x0, x1);
        unpack2(qw[e], y0, y1);
        kk += x0 * x0 + x1 * x1;
        qq += y0 * y0 + y1 * y1;
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
      const float A = expf(bf2f(A_raw));
      const float x = bf2f(pa) + bf2f(dt_raw);
      g_s[st_t] = ok ? -A * (x > 20.0f ? x : logf(1.0f + expf(x))) : 0.f;
      b_s[st_t] = ok ? sigmoidf_(bf2f(pb)) : 0.f;
    }
  }
  lds_barrier();

  // ---- in-chunk cumulative decay and the per-token factors (wave 0). G is summed, differenced and exponentiated
  // in fp64 (exp_nonpos_d): |G| reaches ~50 within a chunk, where an fp32 sum carries ~4e-6 absolute error, and
  // every e^(G_i - G_j) of A and P would inherit it as relative error even between neighbouring tokens (the
  // recurrence applies each token's decay on its own, with no such loss). Emulated in fp64 on the test inputs, the
  // fp32 G alone moves ~3e-4 of the bf16 outputs, against ~2e-5 for the rest of the chunk form in fp32. ----
  if (wave == 0) {
    double x = g_s[lane];
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const double y = __shfl_up(x, d, 64);
      if (lane >= d) x += y;
    }
    const double GC = __shfl(x, 63, 64);
    const float eg = exp_nonpos_d(x);
    G_s[lane] = x;
    fa_s[lane] = b_s[lane] * rk_s[lane];
    vec_g[lane] = eg * rk_s[lane];
    vec_g[CH + lane] = rq_s[lane] * eg;
    vec_g[2 * CH + lane] = rk_s[lane] * exp_nonpos_d(GC - x);
    if (lane != 1) vec_g[3 * CH + lane] = lane == 0 ? exp_nonpos_d(GC) : 0.f;   // lane 1 later: M''s inverse scale
  }

  // ---- Kr Kr^T and Qr Kr^T on the 10 lower 16 x 16 tiles each; tile u of wave w is number w + 4u. Each
  // tile is computed transposed (operands swapped), so a lane holds row 16 I + m16, columns 16 J + 4 g4 .. +3 ----
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
      acc = mma32(*reinterpret_cast<const s16x8*>(brow + 32 * ks), *reinterpret_cast<const s16x8*>(arow + 32 * ks),
                  acc);
    gt[u] = acc;
  }
  lds_barrier();  // per-token factors are in LDS; Qs is free for -A

  // ---- scale the Gram tiles into -A (LDS, fp32) and P (workspace: fp16 hi / lo planes of P 2^sP). Only P's
  // diagonal tiles need the causal mask: the substitution reads A's off-diagonal tiles only and the diagonal
  // inverses read below the diagonal only; P's tiles above the diagonal are never read. |P| <= scale (unit q and
  // k directions, decays <= 1), so its power-of-two scale follows from the scale alone. ----
  {
    float inv_p;
    const float sp = pow2_scale(p.scale, &inv_p);
    float fr[5];
    double Gr[5], Gc[5][4];
    f32x4 rkc[5];
#pragma unroll
    for (int u = 0; u < 5; ++u) {
      const int tau = wave + 4 * u;
      const bool qk = tau >= 10;
      const int idx = qk ? tau - 10 : tau;
      const int I = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
      const int J = idx - I * (I + 1) / 2;
      const int i = 16 * I + m16;
      const int j0 = 16 * J + 4 * g4;
      fr[u] = qk ? rq_s[i] : fa_s[i];
      Gr[u] = G_s[i];
      rkc[u] = ld4f(&rk_s[j0]);
#pragma unroll
      for (int r = 0; r < 4; ++r) Gc[u][r] = G_s[j0 + r];
    }
#pragma unroll
    for (int u = 0; u < 5; ++u) {
      const int tau = wave + 4 * u;
      const bool qk = tau >= 10;
      const int idx = qk ? tau - 10 : tau;
      const int I = idx >= 6 ? 3 : idx >= 3 ? 2 : idx >= 1 ? 1 : 0;
      const int J = idx - I * (I + 1) / 2;
      const int i = 16 * I + m16;
      const int j0 = 16 * J + 4 * g4;
      f32x4 v;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        v[r] = fr[u] * rkc[u][r] * exp_nonpos_d(fmin(Gr[u] - Gc[u][r], 0.0)) * gt[u][r];
        // inside a diagonal tile of P keep row >= column (sign bit of column - row - 1)
        if (qk && I == J) v[r] *= (float)((uint32_t)((4 * g4 + r) - m16 - 1) >> 31);
      }
      if (!qk) {
        *reinterpret_cast<f32x4*>(&nA[i * AS + j0]) = -v;
        if (I == J) *reinterpret_cast<f32x4*>(&Dg[i * DS + 4 * g4]) = -v;
      } else {
        s16x4 vh, vl;
        split4h(v, sp, vh, vl);
        *reinterpret_cast<s16x4*>(&Ph_g[pw_at(i, j0 >> 2)]) = vh;
        *reinterpret_cast<s16x4*>(&Pl_g[pw_at(i, j0 >> 2)]) = vl;
      }
    }
  }
  lds_barrier();  // -A and its diagonal blocks are complete

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
    // every lane group computed the same column; group 0 writes it (constant indices only: a select of t[4 g4 + i]
    // by lane group was lowered to branches over a scratch copy of t and stored row 11 as row 15)
    if (g4 == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) Tf[(wave * 16 + i) * DS + m16] = t[i];
    }
  }
  lds_barrier();  // diagonal inverses are complete

  // ---- M_I = T_II (E_I + sum_{J<I} (-A)_IJ M_J) for this wave's columns 16w + m16 (E = identity), in fp32 on
  // 16x16x4 fp32 MFMAs (lane: row / column m16, k-slot g4). Every operand is read back in B layout by other lanes
  // of the wave, so each block goes through LDS: x_I in the wave's 16 x 16 slice of Dg (free once the diagonal
  // inverses are done), M_I in its 64 x 16 slice of Ks. Each hand-off is a fenced workgroup barrier (all waves run
  // this loop): without an ordering point the compiler may hoist a lane's read of M_J above the stores of other
  // lanes whenever the lane's own store addresses provably differ, and the read then returns the stale x_J.
  // Then M' = M diag(beta). ----
  float* const Mf = reinterpret_cast<float*>(Ks) + wave * (CH * 16);
  float* const Xf = Dg + wave * (16 * DS);
  f32x4 mp[4];
  {
    const float bcol = b_s[16 * wave + m16];
    float amax = 0.f;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int J = 0; J < I; ++J)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          const int k = 16 * J + 4 * j + g4;
          acc = mmf4(nA[(16 * I + m16) * AS + k], Mf[k * 16 + m16], acc);
        }
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        acc[r] += (I == wave && 4 * g4 + r == m16) ? 1.f : 0.f;
        Xf[(4 * g4 + r) * DS + m16] = acc[r];
      }
      lds_barrier();   // x_I is complete (and the previous block's reads of Xf are done)
      f32x4 v = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < 4; ++j)
        v = mmf4(Tf[(16 * I + m16) * DS + 4 * j + g4], Xf[(4 * j + g4) * DS + m16], v);
#pragma unroll
      for (int r = 0; r < 4; ++r) Mf[(16 * I + 4 * g4 + r) * 16 + m16] = v[r];
      lds_barrier();   // M_I is complete before the next block reads it, and x_I has been read
      mp[I] = v * bcol;
      amax = absmax4(mp[I], amax);
    }
    amax = wave_max(amax);
    if (lane == 0) red_s[wave] = amax;
  }
  lds_barrier();  // every wave's M' block is done (Ks is free for the planes) and its largest magnitude is in red_s

  // ---- M' 2^sM as fp16 hi / lo planes, transposed through LDS (the Ks area) into 16-byte stores to the
  // workspace; the inverse scale 2^-sM goes to the factor area ----
  uint16_t* const Mh_s = Ks;
  uint16_t* const Ml_s = Ks + PL;
  {
    float inv_m;
    const float sm = pow2_scale(fmaxf(fmaxf(red_s[0], red_s[1]), fmaxf(red_s[2], red_s[3])), &inv_m);
    if (threadIdx.x == 1) vec_g[3 * CH + 1] = inv_m;
#pragma unroll
    for (int I = 0; I < 4; ++I) {
      s16x4 hi, lo;
      split4h(mp[I], sm, hi, lo);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int at = pw_at(16 * I + 4 * g4 + r, 4 * wave + (m16 >> 2)) + (m16 & 3);
        Mh_s[at] = (uint16_t)hi[r];
        Ml_s[at] = (uint16_t)lo[r];
      }
    }
  }
  lds_barrier();
  // the two planes have the same swizzled rows in LDS and in the workspace: a copy of the lower-triangle slots,
  // all that the state kernel reads (640 of the pair's 1,024 16-byte pieces)
#pragma unroll
  for (int i = 0; i < (2 * TRI_SLOTS + 255) / 256; ++i) {
    const int q = threadIdx.x + 256 * i;
    if (q < 2 * TRI_SLOTS) {
      const int off = tri_slot_offset(q);
      *reinterpret_cast<u32x4*>(Mh_g + off) = *reinterpret_cast<const u32x4*>(Mh_s + off);
    }
  }
}

// ---------------------------------------------------------------------------------------------------------
// Order: the state kernel runs rows with more chunks first (ties by row index). Its workgroups are dispatched in
// this order, so when not all of them fit on the GPU at once, the rows with the longest chunk chains, which
// bound the kernel's duration, start at once instead of after shorter rows.
// ---------------------------------------------------------------------------------------------------------
__global__ __launch_bounds__(1024) void gdn_chunk_order_kernel(const ChunkParams p, int n_rows) {
  __shared__ int nch[ORDER_MAX];
  if (n_rows > ORDER_MAX) {
    for (int j = threadIdx.x; j < n_rows; j += 1024) p.order[j] = j;
    return;
  }
  for (int j = threadIdx.x; j < n_rows; j += 1024) {
    int64_t slot, tok0;
    nch[j] = (row_tokens(p, j, slot, tok0) + CH - 1) / CH;
  }
  __syncthreads();
  for (int j = threadIdx.x; j < n_rows; j += 1024) {
    const int cj = nch[j];
    int rank = 0;
    for (int i = 0; i < n_rows; ++i) {
      const int ci = nch[i];
      rank += (ci > cj) || (ci == cj && i < j);
    }
    p.order[rank] = j;
  }
}

// ---------------------------------------------------------------------------------------------------------
// State: walks one row's chunks in order for one value head and 64 value columns, with 8 waves in two roles.
// Chain waves (0-3) own value columns 16 w .. 16 w + 15 of the block (w = wave & 3), keep S[:, those] in
// accumulator layout and run the products on the state's dependency chain: Y = Kr S, Z, V' = M' Z and the
// state update. Output waves (4-7) compute Q S and O for the same columns from the chain's split S and V',
// handed over through LDS, so those products run beside the chain instead of on it. The next chunk is fetched
// at the top of each chunk (K, M' and the factors by the chain waves, Q, V and P by the output waves) and
// staged at its end, into second buffers where a tile is still being read then (K, P, the factors). Of the
// planes only the lower-triangle blocks are copied. Per chunk:
//   chain:  fetch K M' factors | split S -> Sx | B1 | Y, Z, V' -> Vx      | B2 | W, S update, stage      | B0
//   output: fetch Q V P                        | B1 | Sx -> Q S (64 x 16) | B2 | Vx -> O, stage, store O | B0
// ---------------------------------------------------------------------------------------------------------
constexpr int XP = 64 * 4;         // one handed-over fragment: 64 lanes x 4 bf16

template <typename ST>
__global__ __launch_bounds__(512) void gdn_chunk_state_kernel(const ChunkParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int w = wave & 3;                              // column group of the wave (both roles)
  const bool chain = __builtin_amdgcn_readfirstlane(wave) < 4;   // wave-uniform role
  const int m16 = lane & 15;
  const int g4 = lane >> 4;
  // the two value blocks of one (row, head) are dispatched 8 workgroups apart, i.e. on the same XCD, so
  // their identical K / Q / workspace reads share that XCD's L2
  const int bid = blockIdx.x;
  const int vb = (bid >> 3) & 1;
  const int pair = ((bid >> 4) << 3) | (bid & 7);
  if (pair >= p.pairs) return;
  const int rank = pair / p.HV;
  const int hv = pair - rank * p.HV;
  const int n = p.order[rank];
  const int h = hv / (p.HV / p.H);
  int64_t slot, tok0;
  const int ntok = row_tokens(p, n, slot, tok0);
  const bool padded = p.offsets == nullptr;
  const int vcol = vb * BV + w * 16 + m16;             // this lane's value column (accumulator layout)
  const int64_t ostride = (int64_t)p.HV * VD;

  if (padded) {  // positions past the row's length are zeros in the padded layout
    for (int t = ntok + threadIdx.x / BV; t < p.L; t += 512 / BV) {
      const int64_t at = (tok0 + t) * ostride + hv * VD + vb * BV + (threadIdx.x % BV);
      p.o[at] = 0;
      if (p.sq) p.sq[at] = 0.f;
    }
  }
  if (ntok == 0) return;

  // token-major K (two buffers), Q (swizzled rows, see swz) and V tiles; K^T and the token-column V fragments
  // are read with transpose reads
  __shared__ __align__(16) uint16_t Ks[2][CH * KD];
  __shared__ __align__(16) uint16_t Qs[CH * KD];
  __shared__ __align__(16) uint16_t Vs[CH * VS];
  // M' and P (two buffers) as scaled fp16 hi / lo planes of swizzled token-major rows (lower triangles used)
  __shared__ __align__(16) uint16_t Ms[2 * PL];
  __shared__ __align__(16) uint16_t Ps[2][2 * PL];
  __shared__ __align__(16) float vec_s[2][VEC];
  // hand-over from chain to output waves, in the chain lanes' register layout (lane-linear 8-byte pieces):
  // Sx[w][2 mt + hl] = split S block mt of column group w, Vx[w][2 I + hl] = split V' token block I
  __shared__ __align__(16) uint16_t Sx[4 * 16 * XP];
  __shared__ __align__(16) uint16_t Vx[4 * 8 * XP];
  // the inverse power-of-two scales of the handed-over S and V' fragments, per value column of the block
  __shared__ __align__(16) float s_inv[BV], v_inv[BV];

  // ---- state S[:, vcol] in accumulator layout (chain waves): block mt holds keys 16 mt + 4 g4 + r ----
  ST* sbase = reinterpret_cast<ST*>(p.state) + ((slot * p.HV + hv) * (int64_t)KD) * VD + vcol;
  f32x4 S[8];
  if (chain) {
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) S[mt][r] = load_state<ST>(sbase + (int64_t)(16 * mt + 4 * g4 + r) * VD);
  }

  // ---- swizzled K / Q read offsets (bf16), fixed per lane. Logical piece c of row r sits at c ^ swz(r), and
  // the XOR touches only the low four bits of c, so bit 4 of c (64 bf16) and the row block (16 rows, whose
  // swz is the same) are plain offsets added at the read.
  // yo[2 b + h]: row m16, logical piece g4 + 4 h + 8 b (the row reads of Y and Q S);
  // ko[u]:       row kr = 4 g4 + m16 / 4, logical piece 4 u + m16 % 4 (the transpose reads of K^T). ----
  // po[J]:       plane row m16, logical piece 4 J + g4 (the row reads of M' and P). ----
  int yo[4], ko[4], po[4];
  {
    const int kr = 4 * g4 + (m16 >> 2);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      yo[u] = swz_at(m16, g4 + 4 * (u & 1) + 8 * (u >> 1));
      ko[u] = swz_at(kr, 4 * u + (m16 & 3));
      po[u] = 4 * ((4 * u + g4) ^ swz(m16));
    }
  }

  // ---- staging: thread x of a role (x = threadIdx.x % 256) handles token st_t = x / 4 of the chunk: 16-byte
  // pieces sp + 4 j of its K (chain) or Q (output) row and pieces sp, sp + 4 of its 64 values (output), the
  // lower-triangle plane slots x + 256 i of M' (chain) or P (output) and factor x (chain). Loads are
  // unconditional: a position past the row's end reads the row's first token instead, and its zero factors
  // (rk, rq, and the zero columns of M' and P) cancel it everywhere, so no select can turn into a
  // memory-backed zero or a branch around the loads.
  const int rx = threadIdx.x & 255;
  const int st_t = rx >> 2;
  const int sp = rx & 3;
  // the lower-triangle slots of a plane pair this thread stages (tri_slot_offset)
  int qoff[3];
#pragma unroll
  for (int i = 0; i < 3; ++i) qoff[i] = tri_slot_offset(min(rx + 256 * i, 2 * TRI_SLOTS - 1));
  const bool third = rx + 512 < 2 * TRI_SLOTS;
  auto row_of = [&](int c0) { return p.qkv + (tok0 + (c0 + st_t < ntok ? c0 + st_t : 0)) * p.qkv_stride; };
  // 16-byte piece j of a K / Q row holds logical 8-byte pieces 2j, 2j + 1: it lands in 16-byte slot
  // j ^ (swz >> 1), its halves exchanged when swz is odd. The raw bf16 values are staged as fp16 (exact).
  auto stage_rows = [&](uint16_t* tile, const u32x4* pr) {
    const int sg = swz(st_t);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int at = st_t * KD + 8 * ((sp + 4 * j) ^ (sg >> 1));
      const u32x4 h = bf16x8_to_f16x8(pr[j]);
      *reinterpret_cast<u32x4*>(&tile[at]) = (sg & 1) ? h.zwxy : h;
    }
  };
  uint16_t* const sx = Sx + w * 16 * XP + 4 * lane;
  uint16_t* const vx = Vx + w * 8 * XP + 4 * lane;
  // The two roles run separate loops with the same barriers (three per chunk, after a staging barrier), so
  // the registers of one role are not held across the other's code.
  if (chain) {
    u32x4 pk[4], pm[3];
    float pf;
    auto fetch = [&](int c0) {
      const uint16_t* row = row_of(c0);
      const uint8_t* unit = unit_ptr(p, n, c0 / CH, hv);
#pragma unroll
      for (int j = 0; j < 4; ++j) pk[j] = *reinterpret_cast<const u32x4*>(row + p.k_off + h * KD + 8 * (sp + 4 * j));
#pragma unroll
      for (int i = 0; i < 3; ++i) pm[i] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const uint16_t*>(unit) + qoff[i]);
      pf = reinterpret_cast<const float*>(unit + 4 * PL * 2)[rx];
    };
    auto stage = [&](int buf) {
      stage_rows(Ks[buf], pk);
#pragma unroll
      for (int i = 0; i < 3; ++i)
        if (i < 2 || third) *reinterpret_cast<u32x4*>(Ms + qoff[i]) = pm[i];
      vec_s[buf][rx] = pf;
    };
    fetch(0);
    stage(0);
    lds_barrier();  // B0: chunk 0 staged
    int cb = 0;
    for (int c0 = 0; c0 < ntok; c0 += CH, cb ^= 1) {
      const uint16_t* const K_ = Ks[cb];
      const float* const vec = vec_s[cb];
      // the next chunk (or this one again after the last: staged into idle buffers and never read)
      fetch(c0 + CH < ntok ? c0 + CH : c0);
      // S 2^sS as fp16 hi / lo (sS from the largest |S| of this wave's 16 columns), handed over with 2^-sS
      s16x4 Sh[8], Sl[8];
      float amax = 0.f;
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) amax = absmax4(S[mt], amax);
      float inv_s;
      const float ss = pow2_scale(col_max(amax), &inv_s);
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        split4h(S[mt], ss, Sh[mt], Sl[mt]);
        *reinterpret_cast<s16x4*>(sx + (2 * mt) * XP) = Sh[mt];
        *reinterpret_cast<s16x4*>(sx + (2 * mt + 1) * XP) = Sl[mt];
      }
      if (g4 == 0) s_inv[w * 16 + m16] = inv_s;
      lds_barrier();  // B1: split S handed over

      // ---- Y = Kr S for this wave's 16 value columns: S split hi / lo, key blocks paired ----
      f32x4 Y[4];
      float inv_mz;
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        f32x4 y = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          const int a0 = yo[2 * (q2 & 1)] + 64 * (q2 >> 1) + 16 * I * KD;
          const int a1 = yo[2 * (q2 & 1) + 1] + 64 * (q2 >> 1) + 16 * I * KD;
          const s16x8 ka = cat(ld4h(K_ + a0), ld4h(K_ + a1));
          y = mmh32(ka, cat(Sl[2 * q2], Sl[2 * q2 + 1]), y);
          y = mmh32(ka, cat(Sh[2 * q2], Sh[2 * q2 + 1]), y);
        }
        Y[I] = y * inv_s;
      }
      // ---- Z = Vr - e^G rk . Y, split (V[16 I + 4 g4 + r][column 16 w + m16] by a transpose read) ----
      s16x4 Zh[4], Zl[4];
      {
        const uint16_t* vfrag = Vs + (4 * g4 + (m16 >> 2)) * VS + w * 16 + 4 * (m16 & 3);
        f32x4 z[4];
        float zmax = 0.f;
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          const f32x4 e1 = ld4f(&vec[16 * I + 4 * g4]);
          const s16x4 v4 = ld4h_tr(vfrag + 16 * I * VS);
#pragma unroll
          for (int r = 0; r < 4; ++r) z[I][r] = bf2f((uint16_t)v4[r]) - e1[r] * Y[I][r];
          zmax = absmax4(z[I], zmax);
        }
        float inv_z;
        const float sz = pow2_scale(col_max(zmax), &inv_z);
#pragma unroll
        for (int I = 0; I < 4; ++I) split4h(z[I], sz, Zh[I], Zl[I]);
        inv_mz = vec[3 * CH + 1] * inv_z;   // the M' planes' inverse scale times Z's
      }
      // ---- V'_I = sum_{J<=I} M'_IJ Z_J (M' lower triangular), handed over split ----
      f32x4 Vp[4];
      float vmax = 0.f;
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const uint16_t* mh = Ms + (16 * I + m16) * PW;
        const uint16_t* ml = mh + PL;
        if (I == 0) acc = split_product_sw<1>(mh, ml, po, Zh, Zl, acc);
        if (I == 1) acc = split_product_sw<2>(mh, ml, po, Zh, Zl, acc);
        if (I == 2) acc = split_product_sw<3>(mh, ml, po, Zh, Zl, acc);
        if (I == 3) acc = split_product_sw<4>(mh, ml, po, Zh, Zl, acc);
        Vp[I] = acc * inv_mz;
        vmax = absmax4(Vp[I], vmax);
      }
      {
        float inv_v;
        const float sv = pow2_scale(col_max(vmax), &inv_v);
#pragma unroll
        for (int I = 0; I < 4; ++I) {
          s16x4 vh, vl;
          split4h(Vp[I], sv, vh, vl);
          *reinterpret_cast<s16x4*>(vx + (2 * I) * XP) = vh;
          *reinterpret_cast<s16x4*>(vx + (2 * I + 1) * XP) = vl;
        }
        if (g4 == 0) v_inv[w * 16 + m16] = inv_v;
      }
      lds_barrier();  // B2: split V' handed over; Q, V and M' of this chunk are no longer read

      // ---- S <- e^(G_C) S + Kr^T W,  W = rk e^(G_C - G) . V' (token blocks paired) ----
      s16x4 Wh[4], Wl[4];
      float inv_w;
      {
        f32x4 wv[4];
        float wmax = 0.f;
#pragma unroll
        for (int J = 0; J < 4; ++J) {
          wv[J] = Vp[J] * ld4f(&vec[2 * CH + 16 * J + 4 * g4]);
          wmax = absmax4(wv[J], wmax);
        }
        const float sw = pow2_scale(col_max(wmax), &inv_w);
#pragma unroll
        for (int J = 0; J < 4; ++J) split4h(wv[J], sw, Wh[J], Wl[J]);
      }
      const float gc = vec[3 * CH];
      // K^T operand: lane m16 of group g4 gets key 16 mt + m16 of tokens 16 J + 4 g4 .. +3 (transpose read)
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const int ka0 = ko[mt & 3] + 64 * (mt >> 2);
#pragma unroll
        for (int J = 0; J < 4; J += 2) {
          const s16x8 ka = cat(ld4h_tr(K_ + ka0 + 16 * J * KD), ld4h_tr(K_ + ka0 + 16 * (J + 1) * KD));
          acc = mmh32(ka, cat(Wl[J], Wl[J + 1]), acc);
          acc = mmh32(ka, cat(Wh[J], Wh[J + 1]), acc);
        }
        S[mt] = S[mt] * gc + acc * inv_w;
      }
      stage(cb ^ 1);
      lds_barrier();  // B0: the next chunk is staged
    }
#pragma unroll
    for (int mt = 0; mt < 8; ++mt)
#pragma unroll
      for (int r = 0; r < 4; ++r) store_state(sbase + (int64_t)(16 * mt + 4 * g4 + r) * VD, S[mt][r]);
  } else {
    float inv_p;
    pow2_scale(p.scale, &inv_p);   // the P planes carry P 2^sP (gdn_chunk_prep_kernel)
    u32x4 pq[4], pv[2], pp[3];
    auto fetch = [&](int c0) {
      const uint16_t* row = row_of(c0);
      const uint16_t* unit = reinterpret_cast<const uint16_t*>(unit_ptr(p, n, c0 / CH, hv));
#pragma unroll
      for (int j = 0; j < 4; ++j) pq[j] = *reinterpret_cast<const u32x4*>(row + p.q_off + h * KD + 8 * (sp + 4 * j));
#pragma unroll
      for (int j = 0; j < 2; ++j)
        pv[j] = *reinterpret_cast<const u32x4*>(row + p.v_off + hv * VD + vb * BV + 8 * (sp + 4 * j));
#pragma unroll
      for (int i = 0; i < 3; ++i) pp[i] = *reinterpret_cast<const u32x4*>(unit + 2 * PL + qoff[i]);
    };
    auto stage = [&](int buf) {
      stage_rows(Qs, pq);
#pragma unroll
      for (int j = 0; j < 2; ++j) *reinterpret_cast<u32x4*>(&Vs[st_t * VS + 8 * (sp + 4 * j)]) = pv[j];
#pragma unroll
      for (int i = 0; i < 3; ++i)
        if (i < 2 || third) *reinterpret_cast<u32x4*>(Ps[buf] + qoff[i]) = pp[i];
    };
    fetch(0);
    stage(0);
    lds_barrier();  // B0: chunk 0 staged
    int cb = 0;
    for (int c0 = 0; c0 < ntok; c0 += CH, cb ^= 1) {
      const int nv = min(CH, ntok - c0);
      const float* const vec = vec_s[cb];
      fetch(c0 + CH < ntok ? c0 + CH : c0);
      lds_barrier();  // B1: split S handed over

      // ---- QS^T = S^T Qr^T (value rows, token columns) from the handed-over split S ----
      s16x4 Sh[8], Sl[8];
#pragma unroll
      for (int mt = 0; mt < 8; ++mt) {
        Sh[mt] = *reinterpret_cast<const s16x4*>(sx + (2 * mt) * XP);
        Sl[mt] = *reinterpret_cast<const s16x4*>(sx + (2 * mt + 1) * XP);
      }
      const f32x4 inv_s = ld4f(&s_inv[w * 16 + 4 * g4]);   // the scales of this lane's columns 4 g4 .. +3
      f32x4 X[4];
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        f32x4 qs = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int q2 = 0; q2 < 4; ++q2) {
          const int a0 = yo[2 * (q2 & 1)] + 64 * (q2 >> 1) + 16 * I * KD;
          const int a1 = yo[2 * (q2 & 1) + 1] + 64 * (q2 >> 1) + 16 * I * KD;
          const s16x8 qa = cat(ld4h(Qs + a0), ld4h(Qs + a1));
          qs = mmh32(cat(Sl[2 * q2], Sl[2 * q2 + 1]), qa, qs);
          qs = mmh32(cat(Sh[2 * q2], Sh[2 * q2 + 1]), qa, qs);
        }
        X[I] = qs * inv_s;
      }
      lds_barrier();  // B2: split V' handed over

      // ---- O^T = (QS)^T rq e^G + V'^T P^T: lane holds value columns 4 g4 .. 4 g4 + 3 of token 16 I + m16, so
      // each lane writes one 8-byte piece per token tile ----
      s16x4 Vh[4], Vl[4];
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        Vh[I] = *reinterpret_cast<const s16x4*>(vx + (2 * I) * XP);
        Vl[I] = *reinterpret_cast<const s16x4*>(vx + (2 * I + 1) * XP);
      }
      const f32x4 inv_pv = inv_p * ld4f(&v_inv[w * 16 + 4 * g4]);   // the P planes' and V''s inverse scales
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const int t = 16 * I + m16;
        const float qe = vec[CH + t];
        f32x4 acc = {0.f, 0.f, 0.f, 0.f};
        const uint16_t* ph = Ps[cb] + t * PW;
        const uint16_t* pl = ph + PL;
        if (I == 0) acc = split_product_sw<1, true>(ph, pl, po, Vh, Vl, acc);
        if (I == 1) acc = split_product_sw<2, true>(ph, pl, po, Vh, Vl, acc);
        if (I == 2) acc = split_product_sw<3, true>(ph, pl, po, Vh, Vl, acc);
        if (I == 3) acc = split_product_sw<4, true>(ph, pl, po, Vh, Vl, acc);
        X[I] = X[I] * qe + acc * inv_pv;
      }
      // stage before storing: waiting for the staged loads would also wait for stores issued before it
      stage(cb ^ 1);
#pragma unroll
      for (int I = 0; I < 4; ++I) {
        const int t = 16 * I + m16;
        if (t < nv) {
          const f32x4 o = X[I];
          const int64_t at = (tok0 + c0 + t) * ostride + hv * VD + vb * BV + w * 16 + 4 * g4;
          const uint32_t w01 = pack_bf16x2(o[0], o[1]), w23 = pack_bf16x2(o[2], o[3]);
          *reinterpret_cast<uint2*>(p.o + at) = make_uint2(w01, w23);
          if (p.sq) {
            const float x0 = __uint_as_float(w01 << 16), x1 = __uint_as_float(w01 & 0xffff0000u);
            const float x2 = __uint_as_float(w23 << 16), x3 = __uint_as_float(w23 & 0xffff0000u);
            *reinterpret_cast<f32x4*>(p.sq + at) = (f32x4){x0 * x0, x1 * x1, x2 * x2, x3 * x3};
          }
        }
      }
      lds_barrier();  // B0: the next chunk is staged
    }
  }
}

// Gated RMSNorm of the chunk outputs (gated_finish, src/hs_guard/engine/fused_kernels.py:215-233, as the slot
// step's fused epilogue computes it): one wave per token of a processed row, all value heads (2 values per lane
// each, loads of every head issued together); out = bf16(bf16(w * bf16(o * rsqrt(mean(o^2) + eps))) * silu(z)).
__global__ __launch_bounds__(256) void gdn_chunk_gate_kernel(const ChunkParams p) {
  const int lane = threadIdx.x & 63;
  const int n = blockIdx.y;
  const int t = blockIdx.x * 4 + (threadIdx.x >> 6);
  int64_t slot, tok0;
  const int ntok = row_tokens(p, n, slot, tok0);
  if (t >= ntok) return;
  const int64_t tok = tok0 + t;
  const int64_t ostride = (int64_t)p.HV * VD;
  float w0, w1;
  unpack2(*reinterpret_cast<const uint32_t*>(p.norm_w + 2 * lane), w0, w1);
  for (int hv = 0; hv < p.HV; hv += 4) {
    float x[4][2], zz[4][2];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const int h = min(hv + u, p.HV - 1);
      unpack2(*reinterpret_cast<const uint32_t*>(p.o + tok * ostride + h * VD + 2 * lane), x[u][0], x[u][1]);
      unpack2(*reinterpret_cast<const uint32_t*>(p.z + tok * p.z_stride + h * VD + 2 * lane), zz[u][0], zz[u][1]);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      if (hv + u >= p.HV) break;
      const float r = rsqrtf(wave_sum(x[u][0] * x[u][0] + x[u][1] * x[u][1]) * (1.0f / VD) + p.eps);
      const float y0 = rbf(w0 * rbf(x[u][0] * r)) * siluf_(zz[u][0]);
      const float y1 = rbf(w1 * rbf(x[u][1] * r)) * siluf_(zz[u][1]);
      *reinterpret_cast<uint32_t*>(p.out + tok * ostride + (hv + u) * VD + 2 * lane) =
          (uint32_t)f2bf(y0) | ((uint32_t)f2bf(y1) << 16);
    }
  }
}

}  // namespace
}  // namespace hsg

using hsg::ChunkParams;

namespace {

// Shared argument checks and the two launches (prep, state); returns HSG_OK after launching, or an error code.
int chunk_launch(ChunkParams& p, int32_t state_dtype, int32_t n_rows, int32_t L, int32_t H, int32_t HV, int32_t K,
                 int32_t V, size_t workspace_bytes, hipStream_t s) {
  if (n_rows < 0 || H <= 0 || HV <= 0 || L <= 0 || p.state_rows <= 0) return HSG_ERR_ARG;
  if (!p.qkv || !p.a || !p.b || !p.A_log || !p.dt_bias || !p.state || !p.slots || !p.lens || !p.o || !p.ws)
    return HSG_ERR_ARG;
  if (K != hsg::KD || V != hsg::VD || HV % H != 0) return HSG_ERR_SHAPE;
  if (state_dtype != HSG_STATE_F32 && state_dtype != HSG_STATE_F16) return HSG_ERR_ARG;
  if (!hsg::aligned(p.qkv, 16) || p.qkv_stride % 8 || p.q_off % 8 || p.k_off % 8 || p.v_off % 8) return HSG_ERR_ALIGN;
  if (!hsg::aligned(p.state, 16) || !hsg::aligned(p.o, 8) || (p.sq && !hsg::aligned(p.sq, 16))) return HSG_ERR_ALIGN;
  if (!hsg::aligned(p.ws, 256)) return HSG_ERR_ALIGN;
  p.max_chunks = (L + hsg::CH - 1) / hsg::CH;
  const int64_t units = (int64_t)n_rows * p.max_chunks * HV;
  if ((int64_t)n_rows * HV > (int64_t)1 << 26 || units > (int64_t)0x7fffffff) return HSG_ERR_SHAPE;
  if (workspace_bytes < hsg_gdn_chunk_workspace_bytes(n_rows, L, HV)) return HSG_ERR_SHAPE;
  p.pairs = n_rows * HV;
  p.order = reinterpret_cast<int32_t*>(p.ws + units * hsg::UNIT_BYTES);
  hipLaunchKernelGGL(hsg::gdn_chunk_prep_kernel, dim3((unsigned)units), dim3(256), 0, s, p);
  hipLaunchKernelGGL(hsg::gdn_chunk_order_kernel, dim3(1), dim3(1024), 0, s, p, (int)n_rows);
  const dim3 grid((unsigned)(((p.pairs + 7) / 8) * 16));
  if (state_dtype == HSG_STATE_F32)
    hipLaunchKernelGGL((hsg::gdn_chunk_state_kernel<float>), grid, dim3(512), 0, s, p);
  else
    hipLaunchKernelGGL((hsg::gdn_chunk_state_kernel<uint16_t>), grid, dim3(512), 0, s, p);
  return HSG_OK;
}

ChunkParams chunk_params(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off, int32_t v_off,
                         const void* a, const void* b, int64_t ab_stride, const void* A_log, const void* dt_bias,
                         void* state, int64_t state_rows, const int64_t* slots, const int64_t* lens,
                         const int64_t* offsets, int32_t L, int32_t H, int32_t HV, float scale, void* o, float* sq,
                         int32_t min_len, void* workspace) {
  ChunkParams p{};
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
  p.min_len = min_len;
  p.ws = static_cast<uint8_t*>(workspace);
  return p;
}

}  // namespace

extern "C" size_t hsg_gdn_chunk_workspace_bytes(int32_t n_rows, int32_t L, int32_t HV) {
  if (n_rows <= 0 || L <= 0 || HV <= 0) return 0;
  // the units, then the state kernel's row order (int32 per row, rounded up to 256 bytes)
  return (size_t)n_rows * (size_t)((L + hsg::CH - 1) / hsg::CH) * (size_t)HV * (size_t)hsg::UNIT_BYTES +
         ((size_t)n_rows * 4 + 255) / 256 * 256;
}

extern "C" int hsg_gdn_chunk_prefill(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off,
                                     int32_t v_off, const void* a, const void* b, int64_t ab_stride,
                                     const void* A_log, const void* dt_bias, void* state, int32_t state_dtype,
                                     int64_t state_rows, const int64_t* slots, const int64_t* lens,
                                     const int64_t* offsets, int32_t n_rows, int32_t L, int32_t H, int32_t HV,
                                     int32_t K, int32_t V, float scale, void* o, float* sq, int32_t min_len,
                                     void* workspace, size_t workspace_bytes, void* stream) {
  if (n_rows == 0 && L > 0 && H > 0 && HV > 0 && state_rows > 0) return HSG_OK;
  ChunkParams p = chunk_params(qkv, qkv_stride, q_off, k_off, v_off, a, b, ab_stride, A_log, dt_bias, state,
                               state_rows, slots, lens, offsets, L, H, HV, scale, o, sq, min_len, workspace);
  const int rc = chunk_launch(p, state_dtype, n_rows, L, H, HV, K, V, workspace_bytes,
                              reinterpret_cast<hipStream_t>(stream));
  return rc != HSG_OK ? rc : hsg::launch_status();
}

extern "C" int hsg_gdn_chunk_prefill_gated(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off,
                                           int32_t v_off, const void* a, const void* b, int64_t ab_stride,
                                           const void* A_log, const void* dt_bias, void* state,
                                           int32_t state_dtype, int64_t state_rows, const int64_t* slots,
                                           const int64_t* lens, const int64_t* offsets, int32_t n_rows, int32_t L,
                                           int32_t H, int32_t HV, int32_t K, int32_t V, float scale, void* o,
                                           const void* z, int64_t z_stride, const void* norm_w, float eps,
                                           void* out, int32_t min_len, void* workspace, size_t workspace_bytes,
                                           void* stream) {
  if (n_rows == 0 && L > 0 && H > 0 && HV > 0 && state_rows > 0) return HSG_OK;
  if (!z || !norm_w || !out || offsets == nullptr) return HSG_ERR_ARG;   // packed layout only
  if (!hsg::aligned(z, 4) || z_stride % 2 || !hsg::aligned(norm_w, 4) || !hsg::aligned(out, 4)) return HSG_ERR_ALIGN;
  ChunkParams p = chunk_params(qkv, qkv_stride, q_off, k_off, v_off, a, b, ab_stride, A_log, dt_bias, state,
                               state_rows, slots, lens, offsets, L, H, HV, scale, o, nullptr, min_len, workspace);
  p.z = static_cast<const uint16_t*>(z);
  p.z_stride = z_stride;
  p.norm_w = static_cast<const uint16_t*>(norm_w);
  p.eps = eps;
  p.out = static_cast<uint16_t*>(out);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const int rc = chunk_launch(p, state_dtype, n_rows, L, H, HV, K, V, workspace_bytes, s);
  if (rc != HSG_OK) return rc;
  hipLaunchKernelGGL(hsg::gdn_chunk_gate_kernel, dim3((unsigned)((L + 3) / 4), (unsigned)n_rows), dim3(256), 0, s, p);
  return hsg::launch_status();
}
