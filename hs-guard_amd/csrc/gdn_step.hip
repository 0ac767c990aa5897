// Gated-delta-rule recurrent slot step for gfx950.
//
// Recurrence (per row n, value head hv, real token t), as src/hs_guard/engine/fused_kernels.py:166-188:
//   q <- q / sqrt(|q|^2 + 1e-6) * scale,  k <- k / sqrt(|k|^2 + 1e-6)
//   g = -exp(A_log) * softplus(a + dt_bias)   (threshold 20),  beta = sigmoid(b)
//   S <- exp(g) S;  v' = beta (v - S^T k);  S <- S + k v'^T;  o = S^T q
//
// Mapping: one 256-thread workgroup per (row, value head); wave w owns value columns [32w, 32w+32).
// Lane (c = lane & 7, rg = lane >> 3) holds the 16 x 4 block S[16rg .. 16rg+15][32w+4c .. +3] in
// registers for the whole tick, so the 64 KiB fp32 state of a (slot, head) is read once and written once
// per tick whatever the token count. Each state load is a 16-byte vector; the 8 lanes of one rg cover a
// 128-byte row segment, so every load instruction reads 8 full 128-byte lines. The k.S and q.S
// reductions over the 128 key rows are in-lane (16 rows) plus a 3-step butterfly over rg (lane xor 8,
// 16, 32) done with a DPP row rotate and gfx950's permlane16/32 swaps, not the LDS crossbar. The state is
// read with nontemporal loads and written back with nontemporal stores (it is touched once per tick). In a
// step each layer's state was last touched a whole step earlier, so its reads miss the 256 MB Infinity Cache;
// measured on MI355X with three state buffers in rotation, 352 x 1: nontemporal loads 142.9 us, ordinary loads
// 159.1 us (ordinary loads win only when one buffer is reused back to back, 129 vs 142 us, which no step does).
// Per-token work is cut to the three 16 x 4 products a token needs (S^T k, the rank-1 update, S^T q):
//   * the registers hold St with S = D St, so exp(g) scales the scalar D, not 64 registers (D is folded
//     back before 1 / D could overflow and when the state is stored);
//   * token inputs (q, k of the key head; v, z of the value head; a, b) arrive in bursts of CT tokens by
//     one cooperative round of 16-byte loads, prefetched into registers one burst ahead; when a burst
//     moves into LDS its q and k are L2-normalised once per token (not once per lane) and exp(g) and
//     beta are computed once per token;
//   * the gated RMSNorm epilogue runs once per burst on all 256 threads, so the token loop has no barrier.
#include "hsg_common.h"

namespace hsg {
namespace {

constexpr int KD = 128;
constexpr int VD = 128;
constexpr int TILE_V = 32;
constexpr int ROWS = 16;
constexpr int CT = 8;    // tokens staged in LDS per burst (the next burst is prefetched into registers)

struct GdnParams {
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
  float scale;
  uint16_t* o;
  float* sq;
  const uint16_t* z;
  int64_t z_stride;
  const uint16_t* norm_w;
  float eps;
  uint16_t* out;
  int skip_rows, skip_min_len;   // packed layout: rows n < skip_rows with lens >= skip_min_len are left alone
  int mfma_min;                  // rows of at least this many tokens take the MFMA burst path (0: none)
  // fused causal conv (CONV): qkv holds the raw projection; weights [conv_C, 4], history pool [state_rows, 3, conv_C]
  const uint16_t* conv_w;
  uint16_t* conv_pool;
  int conv_C;
};

template <typename ST>
struct StateIO;

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <>
struct StateIO<float> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    const f32x4_t x = __builtin_nontemporal_load(reinterpret_cast<const f32x4_t*>(p));
    v[0] = x[0]; v[1] = x[1]; v[2] = x[2]; v[3] = x[3];
  }
  static __device__ __forceinline__ void store(float* p, const float* v) {
    const f32x4_t x = {v[0], v[1], v[2], v[3]};
    __builtin_nontemporal_store(x, reinterpret_cast<f32x4_t*>(p));
  }
};

template <>
struct StateIO<uint16_t> {  // fp16 storage, fp32 arithmetic
  static __device__ __forceinline__ void load(const uint16_t* p, float* v) {
    const u32x2_t w = __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(p));
    v[0] = h2f((uint16_t)(w[0] & 0xffffu)); v[1] = h2f((uint16_t)(w[0] >> 16));
    v[2] = h2f((uint16_t)(w[1] & 0xffffu)); v[3] = h2f((uint16_t)(w[1] >> 16));
  }
  static __device__ __forceinline__ void store(uint16_t* p, const float* v) {
    u32x2_t w;
    w[0] = (uint32_t)f2h(v[0]) | ((uint32_t)f2h(v[1]) << 16);
    w[1] = (uint32_t)f2h(v[2]) | ((uint32_t)f2h(v[3]) << 16);
    __builtin_nontemporal_store(w, reinterpret_cast<u32x2_t*>(p));
  }
};

// Sum over the 8 lanes sharing (lane & 7): lane xor 8, 16, 32 (DPP row rotate, then the two permlane swaps).
__device__ __forceinline__ float sum_rg(float x) { return sum_stride8_dpp(x); }

constexpr int CKS = 4;            // conv taps
constexpr int CH3 = 3 * KD;       // conv channels of one (row, value head) workgroup: q and k of its key head, v

// Dispatch order of the rows. The engine packs rows longest first, and workgroups start in blockIdx order, so
// in plain order the first ~768 resident workgroups (3 per CU) would all be multi-token rows running their
// token chains while HBM idles. Position i of the dispatch order instead takes one row in ROW_MIX from the
// front (long) end of the list and the others from the back (short) end, so each CU streams state beside a
// token chain. ROW_MIX is odd: a row's 16 workgroups land on local slots 2i, 2i + 1 of every XCD, and with an
// even factor the long rows would fall on a fixed subset of CUs. Measured on a config-5 tick: 5 beats 3, 7,
// 9 and 11, and plain order is 10 % slower.
constexpr int ROW_MIX = 5;
__device__ __forceinline__ int dispatch_row(int i, int n_rows) {
  const int q = i / ROW_MIX, m = i - q * ROW_MIX;
  return m == 0 ? q : n_rows - 1 - (q * (ROW_MIX - 1) + m - 1);
}

template <typename ST, bool GATED, bool CONV>
__global__ __launch_bounds__(256) void gdn_step_kernel(const GdnParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 7;
  const int rg = lane >> 3;
  const int ib = blockIdx.x / p.HV;
  const int hv = blockIdx.x - ib * p.HV;
  const int n = dispatch_row(ib, gridDim.x / p.HV);
  const int h = hv / (p.HV / p.H);
  // The row's slot, length and token offset are read together (padded: lens stands in for the offset, unused)
  // and checked without short-circuit branches: each branch made the compiler wait for one value before issuing
  // the next read, three dependent round trips before the first burst's loads.
  const bool padded = p.offsets == nullptr;
  const int64_t slot = p.slots[n];
  const int64_t len_n = p.lens[n];
  const int64_t off_n = (padded ? p.lens : p.offsets)[n];
  int ntok = (int)len_n;
  const bool rejected = (slot < 0) | (slot >= p.state_rows) | (ntok < 0);
  const bool chunked = !padded & (n < p.skip_rows) & (ntok >= p.skip_min_len);   // routed to the chunk kernels
  ntok = (rejected | chunked) ? 0 : padded ? min(ntok, p.L) : ntok;   // padded: never past its L positions
  const int64_t tok0 = padded ? (int64_t)n * p.L : off_n;
  const int col = wave * TILE_V + c * 4;
  // padded layout: the row's outputs at positions t >= ntok are zeros
  auto zero_tail = [&]() __attribute__((always_inline)) {
    if (!padded || rg != 0) return;
    const float zero[4] = {0.f, 0.f, 0.f, 0.f};
    for (int t = ntok; t < p.L; ++t) {
      const int64_t tok = tok0 + t;
      if constexpr (!GATED) {
        const int64_t base = (tok * p.HV + hv) * VD + col;
        store4_bf16(p.o + base, zero);
        if (p.sq != nullptr) *reinterpret_cast<float4*>(p.sq + base) = make_float4(0.f, 0.f, 0.f, 0.f);
      } else {
        store4_bf16(p.out + tok * (int64_t)(p.HV * VD) + hv * VD + col, zero);
      }
    }
  };
  if (ntok == 0) {   // uniform over the workgroup; nothing is read or updated
    zero_tail();
    return;
  }

  // The registers hold St with S = D * St: the per-token decay multiplies the scalar D instead of all 64
  // registers; D is folded back into St before 1 / D could overflow and when the state is stored.
  float S[ROWS][4];
  float D = 1.0f;
  ST* sp = reinterpret_cast<ST*>(p.state) + ((slot * p.HV + hv) * KD + rg * ROWS) * (int64_t)VD + col;
  // the head's decay parameters, read here and converted where the staging uses them, so their wait falls after
  // the first burst's loads are issued instead of before
  const uint16_t a_log_h = p.A_log[hv], dt_h = p.dt_bias[hv];
  // per burst: normalised q (times scale) and k in fp32, one 16-row piece per lane group (stride 20 floats, so
  // the 8 pieces a wave reads at once fall on distinct banks); raw v and z; exp(g) and beta per token
  __shared__ __align__(16) float fq_[CT][KD / ROWS][ROWS + 4];
  __shared__ __align__(16) float fk_[CT][KD / ROWS][ROWS + 4];
  __shared__ __align__(16) uint16_t sv_[CT][VD];
  __shared__ __align__(16) uint16_t sz_[GATED ? CT : 1][VD];
  __shared__ __align__(16) float so_[CT][VD];   // bf16-rounded o of the burst (gated norm; the burst path's outputs)
  __shared__ float sdec_[CT], sbe_[CT];
  constexpr int SEGS = GATED ? 64 : 48;   // 16-byte segments per token: q, k, v (, z)
  // CONV: the burst's raw q, k, v rows (48 segments each), then its z rows; the first burst also fetches the 3
  // raw rows before it (the conv history pool), later bursts take them from the previous burst's raw rows in LDS
  constexpr int RAWSEG0 = (CT + CKS - 1) * 48, RAWSEG = CT * 48;
  constexpr int NSEG0 = CONV ? RAWSEG0 + CT * 16 : CT * SEGS;
  constexpr int NSEG = CONV ? RAWSEG + CT * 16 : CT * SEGS;
  constexpr int PF = (NSEG + 255) / 256;    // segments per thread per burst (the last partly idle)
  constexpr int PF0 = (NSEG0 + 255) / 256;  // the same for the first burst
  // CONV: raw rows (row r = token t0 + r - 3 of the burst), conv + SiLU outputs of the burst, tap weights
  __shared__ __align__(16) uint16_t rw_[CONV ? CT + CKS - 1 : 1][CONV ? CH3 : 8];
  __shared__ __align__(16) uint16_t co_[CONV ? CT : 1][CONV ? CH3 : 8];
  __shared__ __align__(16) uint16_t cw_[CONV ? CH3 : 1][CKS];
  // conv channel of local channel lc (q of key head h, then its k, then v of value head hv)
  auto conv_ch = [&](int lc) {
    return lc < KD ? p.q_off + h * KD + lc : lc < 2 * KD ? p.k_off + h * KD + lc - KD : p.v_off + hv * VD + lc - 2 * KD;
  };
  // gated-norm weights staged in LDS once (read per token from global memory they were reloaded after every
  // output store, since `out` may alias them: one global round trip per token)
  __shared__ __align__(16) uint16_t sw_[GATED ? VD : 1];

  // The tokens of a row go through LDS in bursts of CT; the next burst is loaded into registers while the
  // current one is processed. Segment e = threadIdx.x + 256 i of a burst is token e / SEGS, piece e % SEGS
  // (pieces 16j .. 16j+15 are q, k, v, z for j = 0..3: an aligned group of 16 lanes holds one whole vector);
  // positions past the row's end re-read its last token (never stored to LDS).
  u32x4 pf[PF], pf0[CONV ? PF0 : 1];
  uint16_t pa = 0, pb = 0;
  // CONV, first burst: raw row r = token r - 3 (negative: conv history pool row r), then the z rows
  auto fetch_first_conv = [&]() __attribute__((always_inline)) {
    const int tid = tid_per_site();
#pragma unroll
    for (int i = 0; i < PF0; ++i) {
      const int e = min((int)tid + 256 * i, NSEG0 - 1);
      const uint16_t* src;
      if (e < RAWSEG0) {
        const int r = e / 48, gc = conv_ch((e % 48) * 8);
        src = r < CKS - 1 ? p.conv_pool + (slot * (CKS - 1) + r) * (int64_t)p.conv_C + gc
                          : p.qkv + (tok0 + min(r - (CKS - 1), ntok - 1)) * p.qkv_stride + gc;
      } else {
        const int u = min((e - RAWSEG0) / 16, ntok - 1);
        src = p.z + (tok0 + u) * p.z_stride + hv * VD + ((e - RAWSEG0) & 15) * 8;
      }
      pf0[CONV ? i : 0] = *reinterpret_cast<const u32x4*>(src);
    }
    const int64_t tok = tok0 + min((int)tid, ntok - 1);
    pa = p.a[tok * p.ab_stride + hv];
    pb = p.b[tok * p.ab_stride + hv];
  };
  auto fetch = [&](int t) __attribute__((always_inline)) {
    const int tid = tid_per_site();
    const int last = ntok - 1 - t;
    if constexpr (CONV) {   // raw rows of tokens t .. t + 7, then their z rows
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int e = tid + 256 * i;
        const uint16_t* src;
        if (e < RAWSEG) {
          const int u = min(e / 48, last);
          src = p.qkv + (tok0 + t + u) * p.qkv_stride + conv_ch((e % 48) * 8);
        } else {
          const int u = min((e - RAWSEG) / 16, last);
          src = p.z + (tok0 + t + u) * p.z_stride + hv * VD + ((e - RAWSEG) & 15) * 8;
        }
        pf[i] = *reinterpret_cast<const u32x4*>(src);
      }
      const int64_t tok = tok0 + t + min((int)tid, last);
      pa = p.a[tok * p.ab_stride + hv];
      pb = p.b[tok * p.ab_stride + hv];
      return;
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int e = tid + 256 * i;
      const int u = min(e / SEGS, last);
      const int sg = e % SEGS;
      const int which = sg >> 4;
      const int c = (sg & 15) * 8;
      const int64_t tok = tok0 + t + u;
      const uint16_t* row = p.qkv + tok * p.qkv_stride;
      const uint16_t* src = which == 0 ? row + p.q_off + h * KD + c
                          : which == 1 ? row + p.k_off + h * KD + c
                          : which == 2 ? row + p.v_off + hv * VD + c
                                       : p.z + tok * p.z_stride + hv * VD + c;
      pf[i] = *reinterpret_cast<const u32x4*>(src);
    }
    const int64_t tok = tok0 + t + min((int)tid, last);
    pa = p.a[tok * p.ab_stride + hv];
    pb = p.b[tok * p.ab_stride + hv];
  };
  // prefetched burst -> LDS: q <- q / sqrt(|q|^2 + 1e-6) * scale and k <- k / sqrt(|k|^2 + 1e-6) once per token
  // (|x|^2 summed over the 16 lanes holding the vector), v and z as loaded, exp(g) and beta by thread u
  // CONV: raw rows -> LDS, then each (token, 4 channels) of the burst gets acc = sum_k w[c, k] x[t - 3 + k] in
  // fp32 (as conv_silu_kernel) and bf16(silu(bf16(acc))), then q and k are normalised from those outputs
  // (later bursts: hist holds the previous burst's raw rows CT .. CT + 2, read by threads < 144)
  u32x4 hist;
  auto stage_conv = [&](int nt, bool first) __attribute__((always_inline)) {
    const int tid = tid_per_site();
    if (first) {
#pragma unroll
      for (int i = 0; i < PF0; ++i) {
        const int e = tid + 256 * i;
        if (e < RAWSEG0) {
          const int r = e / 48;
          if (r < nt + CKS - 1) *reinterpret_cast<u32x4*>(&rw_[CONV ? r : 0][(e % 48) * 8]) = pf0[CONV ? i : 0];
        } else if (e < NSEG0) {
          const int u = (e - RAWSEG0) / 16;
          if (u < nt) *reinterpret_cast<u32x4*>(&sz_[GATED ? u : 0][((e - RAWSEG0) & 15) * 8]) = pf0[CONV ? i : 0];
        }
      }
    } else {
      if (tid < (CKS - 1) * 48)
        *reinterpret_cast<u32x4*>(&rw_[CONV ? tid / 48 : 0][(tid % 48) * 8]) = hist;
#pragma unroll
      for (int i = 0; i < PF; ++i) {
        const int e = tid + 256 * i;
        if (e < RAWSEG) {
          const int u = e / 48;
          if (u < nt) *reinterpret_cast<u32x4*>(&rw_[CONV ? u + CKS - 1 : 0][(e % 48) * 8]) = pf[i];
        } else {
          const int u = (e - RAWSEG) / 16;
          if (u < nt) *reinterpret_cast<u32x4*>(&sz_[GATED ? u : 0][((e - RAWSEG) & 15) * 8]) = pf[i];
        }
      }
    }
    __syncthreads();
    // items of 4 channels of one token: CT * 96 of them, 3 per thread at CT = 8, so every wave has the same
    // share (items of 8 channels gave two waves twice the work of the other two)
#pragma unroll
    for (int i = 0; i < (CT * 96 + 255) / 256; ++i) {
      const int item = tid + 256 * i;
      const int u = item / 96, c0 = (item % 96) * 4;
      if (u < nt) {
        u32x2 xr[CKS];
#pragma unroll
        for (int k = 0; k < CKS; ++k) xr[k] = *reinterpret_cast<const u32x2*>(&rw_[CONV ? u + k : 0][c0]);
        u32x2 y;
#pragma unroll
        for (int j = 0; j < 4; j += 2) {
          float rr[2];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {
            const uint2 wv = *reinterpret_cast<const uint2*>(&cw_[CONV ? c0 + j + hh : 0][0]);
            float w4[4];
            unpack2(wv.x, w4[0], w4[1]);
            unpack2(wv.y, w4[2], w4[3]);
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < CKS; ++k) {
              const uint32_t word = xr[k][(j + hh) >> 1];
              acc = fmaf(w4[k], __uint_as_float(((j + hh) & 1) ? (word & 0xffff0000u) : (word << 16)), acc);
            }
            rr[hh] = siluf_(rbf(acc));
          }
          y[j >> 1] = (uint32_t)f2bf(rr[0]) | ((uint32_t)f2bf(rr[1]) << 16);
        }
        *reinterpret_cast<u32x2*>(&co_[CONV ? u : 0][c0]) = y;
      }
    }
    __syncthreads();
    {  // q, k of the burst: 8 tokens x 32 segments, one per thread
      const int e = tid;
      const int u = e >> 5, which = (e >> 4) & 1, c = (e & 15) * 8;
      const u32x4 v = *reinterpret_cast<const u32x4*>(&co_[CONV ? u : 0][which * KD + c]);
      float x[8];
      unpack2(v[0], x[0], x[1]);
      unpack2(v[1], x[2], x[3]);
      unpack2(v[2], x[4], x[5]);
      unpack2(v[3], x[6], x[7]);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
      ss = sum16_dpp(ss);
      if (u < nt) {
        const float r = 1.0f / sqrtf(ss + 1e-6f);
        f32x4_t y0, y1;
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          y0[j] = which == 0 ? x[j] * r * p.scale : x[j] * r;
          y1[j] = which == 0 ? x[4 + j] * r * p.scale : x[4 + j] * r;
        }
        float* dst = which == 0 ? &fq_[u][c / ROWS][c % ROWS] : &fk_[u][c / ROWS][c % ROWS];
        *reinterpret_cast<f32x4_t*>(dst) = y0;
        *reinterpret_cast<f32x4_t*>(dst + 4) = y1;
      }
    }
    if (tid < nt) {
      uint32_t al = a_log_h, dh = dt_h;
      asm volatile("" : "+v"(al), "+v"(dh));   // an empty fence: the conversion below is not hoisted above here
      const float x = bf2f((uint16_t)pa) + bf2f((uint16_t)dh);
      const float g = -expf(bf2f((uint16_t)al)) * (x > 20.0f ? x : logf(1.0f + expf(x)));
      sdec_[tid] = expf(g);
      sbe_[tid] = sigmoidf_(bf2f(pb));
    }
  };
  auto stage = [&](int nt, bool first) __attribute__((always_inline)) {
    const int tid = tid_per_site();
    if constexpr (CONV) {
      stage_conv(nt, first);
      return;
    }
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int e = tid + 256 * i;
      const int u = e / SEGS;
      const int sg = e % SEGS;
      const int which = sg >> 4;
      const int c = (sg & 15) * 8;
      float x[8];
      unpack2(pf[i][0], x[0], x[1]);
      unpack2(pf[i][1], x[2], x[3]);
      unpack2(pf[i][2], x[4], x[5]);
      unpack2(pf[i][3], x[6], x[7]);
      float ss = 0.f;
#pragma unroll
      for (int j = 0; j < 8; ++j) ss += x[j] * x[j];
      ss = sum16_dpp(ss);
      if (u < nt) {
        if (which < 2) {
          const float r = 1.0f / sqrtf(ss + 1e-6f);
          f32x4_t y0, y1;
          if (which == 0) {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              y0[j] = x[j] * r * p.scale;
              y1[j] = x[4 + j] * r * p.scale;
            }
          } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) {
              y0[j] = x[j] * r;
              y1[j] = x[4 + j] * r;
            }
          }
          float* dst = which == 0 ? &fq_[u][c / ROWS][c % ROWS] : &fk_[u][c / ROWS][c % ROWS];
          *reinterpret_cast<f32x4_t*>(dst) = y0;
          *reinterpret_cast<f32x4_t*>(dst + 4) = y1;
        } else if (which == 2) {
          *reinterpret_cast<u32x4*>(&sv_[u][c]) = pf[i];
        } else if (GATED) {
          *reinterpret_cast<u32x4*>(&sz_[GATED ? u : 0][c]) = pf[i];
        }
      }
    }
    if (tid < nt) {
      uint32_t al = a_log_h, dh = dt_h;
      asm volatile("" : "+v"(al), "+v"(dh));   // an empty fence: the conversion below is not hoisted above here
      const float x = bf2f((uint16_t)pa) + bf2f((uint16_t)dh);
      const float g = -expf(bf2f((uint16_t)al)) * (x > 20.0f ? x : logf(1.0f + expf(x)));
      sdec_[tid] = expf(g);
      sbe_[tid] = sigmoidf_(bf2f(pb));
    }
  };
  // gated RMSNorm of the burst's outputs (so_, bf16-rounded o), stored to `out`: 32 threads per token, 4 value
  // columns each
  auto gated_epilogue = [&](int t0, int nt) __attribute__((always_inline)) {
    __syncthreads();
    const int u = threadIdx.x >> 5;
    const int cc = (threadIdx.x & 31) * 4;
    const f32x4_t ob = *reinterpret_cast<const f32x4_t*>(&so_[u][cc]);
    float part = 0.f;
#pragma unroll
    for (int i = 0; i < 4; ++i) part += ob[i] * ob[i];
    part = sum32_dpp(part);
    const float r = rsqrtf(part * (1.0f / VD) + p.eps);
    if (u < nt) {
      float y[4], z4[4], w4[4];
      load4_bf16(&sz_[GATED ? u : 0][cc], z4);
      load4_bf16(&sw_[GATED ? cc : 0], w4);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float hb = rbf(ob[i] * r);
        const float tw = rbf(w4[i] * hb);
        y[i] = tw * siluf_(z4[i]);
      }
      store4_bf16(p.out + (tok0 + t0 + u) * (int64_t)(p.HV * VD) + hv * VD + cc, y);
    }
  };
  // the next burst into LDS once every read of this one is done
  auto next_burst = [&](int t0) __attribute__((always_inline)) {
    // the next burst's conv history: this (full) burst's last 3 raw rows
    if (CONV && threadIdx.x < (CKS - 1) * 48)
      hist = *reinterpret_cast<const u32x4*>(&rw_[CONV ? CT + threadIdx.x / 48 : 0][(threadIdx.x % 48) * 8]);
    __syncthreads();
    stage(min(CT, ntok - t0 - CT), false);
  };
  auto store_conv_history = [&]() __attribute__((always_inline)) {
    if (CONV && threadIdx.x < (CKS - 1) * 48) {
      // new conv history = ext[ntok .. ntok + 2] of ext = [pool; tokens]: raw rows nt .. nt + 2 of the last burst
      // (the row's last three tokens, or old pool rows when it has fewer); every read of the old rows came first
      const int nt_last = ntok - (ntok - 1) / CT * CT;
      const int i = threadIdx.x / 48, sg = threadIdx.x % 48;
      *reinterpret_cast<u32x4*>(p.conv_pool + (slot * (CKS - 1) + i) * (int64_t)p.conv_C + conv_ch(8 * sg)) =
          *reinterpret_cast<const u32x4*>(&rw_[CONV ? nt_last + i : 0][8 * sg]);
    }
  };

  // ---------------------------------------------------------------------------------------------------------
  // Burst path, for rows of at least p.mfma_min tokens: each burst of CT tokens in the WY/UT chunk form on fp32
  // MFMA (v_mfma_f32_16x16x4f32) instead of CT dependent token updates on the VALU. With Gamma_t the decay from
  // the burst's start through token t, X = K S0, Y = Q S0 (one product: K and Q stacked as the 16 rows of one
  // operand), A[t][s] = beta_t Gamma_t / Gamma_s (k_t . k_s) for s < t, T = (I + A)^-1:
  //   V' = T diag(beta) (V - diag(Gamma) X),  O = diag(Gamma) Y + (Gamma_t / Gamma_s (q_t . k_s))_{s<=t} V',
  //   S_C = Gamma_C S0 + K^T diag(Gamma_C / Gamma) V'
  // (the token recurrence unrolled; equal in exact arithmetic). The state stays in registers in the MFMA
  // accumulator layout, as St with S = D St (D folded back as in the token path): wave w owns value columns
  // [32w, 32w + 32) as 16 tiles of 16 keys x 16 columns; lane (j4 = lane / 16, n16 = lane % 16) holds
  // Sm[2 kt + ct][i] = St[16 kt + 4 j4 + i][32 w + 16 ct + n16]. In X = K St that is the B operand as it stands
  // (the contraction index of step (kt, i), slot j4, is key 16 kt + 4 j4 + i), and the update K^T W accumulates
  // onto it. Staging, the conv, the gated norm and the conv history are the token path's.
  // ---------------------------------------------------------------------------------------------------------
  if (p.mfma_min > 0 && ntok >= p.mfma_min) {   // uniform over the workgroup
    __shared__ __align__(16) float gp_[4][CT][2 * CT];   // per-wave partial Gram rows: K k^T (t < CT), Q k^T
    __shared__ __align__(16) float am_[CT][CT], tm_[CT][CT], bm_[CT][CT], fac_[2][CT];
    // the (slot, head) state block as a buffer resource: every state load and store is one VGPR lane offset,
    // the key tile's offset as a scalar and the rest as an immediate (no per-access 64-bit addresses, which the
    // compiler would otherwise compute up front and keep live across the bursts)
    const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc(
        reinterpret_cast<ST*>(p.state) + (slot * p.HV + hv) * (int64_t)(KD * VD), (short)0,
        (int)(KD * VD * sizeof(ST)), 0x00020000);
    // token index of contraction slot k at step s of an 8-token contraction: lanes 0-31 take their own rows
    // 4 k + 2 s, lanes 32-63 rows 4 (k - 2) + 2 s + 1 through permlane32_swap (see bop)
    auto tau = [](int s, int k) { return 4 * (k & 1) + 2 * s + (k >> 1); };
    // B operand of an 8-token contraction from a D-layout value (rows 4 j4 + i): lanes 0-31 keep register 2 s,
    // lanes 32-63 receive register 2 s + 1 of lane - 32
    auto bop = [](const f32x4_t& x, int s) {
      return __uint_as_float(__builtin_amdgcn_permlane32_swap(__float_as_uint(x[2 * s]), __float_as_uint(x[2 * s + 1]),
                                                              false, false)[0]);
    };
    // zero the K and Q rows of a partial burst's missing tokens (products with them must be exactly zero)
    auto zero_pad = [&](int nt) __attribute__((always_inline)) {
      for (int e = threadIdx.x; e < (CT - nt) * KD; e += 256) {
        const int u = nt + e / KD, cc = e % KD;
        fq_[u][cc / ROWS][cc % ROWS] = 0.f;
        fk_[u][cc / ROWS][cc % ROWS] = 0.f;
      }
    };
    if constexpr (CONV) fetch_first_conv();
    else fetch(0);
    u32x4 cwr[4], swr;
    if constexpr (CONV) {
      const uint16_t* wsrc = p.conv_w + (int64_t)conv_ch(8 * min((int)threadIdx.x, CH3 / 8 - 1)) * CKS;
#pragma unroll
      for (int j = 0; j < 4; ++j) cwr[j] = *reinterpret_cast<const u32x4*>(wsrc + 8 * j);
    }
    if constexpr (GATED) swr = *reinterpret_cast<const u32x4*>(p.norm_w + 8 * min((int)threadIdx.x, VD / 8 - 1));
    __builtin_amdgcn_sched_barrier(0);
    const int soff = (4 * (lane >> 4) * VD + wave * TILE_V + (lane & 15)) * (int)sizeof(ST);   // lane's byte offset
    constexpr int KT_BYTES = 16 * VD * (int)sizeof(ST);
    f32x4_t Sm[16];
#pragma unroll
    for (int kt = 0; kt < KD / 16; ++kt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int off = soff + (i * VD + 16 * ct) * (int)sizeof(ST);
          if constexpr (sizeof(ST) == 4)
            Sm[2 * kt + ct][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, off, kt * KT_BYTES, 2));
          else
            Sm[2 * kt + ct][i] = h2f(__builtin_amdgcn_raw_buffer_load_b16(srs, off, kt * KT_BYTES, 2));
        }
    if (CONV && threadIdx.x < CH3 / 8) {
#pragma unroll
      for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(&cw_[CONV ? 8 * threadIdx.x : 0][0] + 8 * j) = cwr[j];
    }
    if (GATED && threadIdx.x < VD / 8) *reinterpret_cast<u32x4*>(&sw_[GATED ? 8 * threadIdx.x : 0]) = swr;
    float D = 1.0f;
    stage(min(CT, ntok), true);
    zero_pad(min(CT, ntok));
    for (int t0 = 0; t0 < ntok; t0 += CT) {
      const int nt = min(CT, ntok - t0);
      if (t0 + CT < ntok) fetch(t0 + CT);
      __syncthreads();
      // lane indices of this burst's products, recomputed here (not hoisted out of the loop: every address
      // derived from them would otherwise stay live across the next burst's staging)
      const int bt = tid_per_site();
      const int j4 = (bt & 63) >> 4, n16 = bt & 15;
      const int cbase = (bt >> 6) * TILE_V + n16;
      // X = K St (rows 0-7) and Y = Q St (rows 8-15); this wave's share of the Gram products [K; Q] K^T
      f32x4_t xy[2] = {{0.f, 0.f, 0.f, 0.f}, {0.f, 0.f, 0.f, 0.f}};
      f32x4_t gr = {0.f, 0.f, 0.f, 0.f};
      const float* arow = n16 < CT ? &fk_[n16 & (CT - 1)][0][4 * j4] : &fq_[n16 & (CT - 1)][0][4 * j4];
#pragma unroll
      for (int kt = 0; kt < KD / 16; ++kt) {
        const f32x4_t a4 = *reinterpret_cast<const f32x4_t*>(arow + kt * (ROWS + 4));
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          xy[0] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i], Sm[2 * kt][i], xy[0], 0, 0, 0);
          xy[1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i], Sm[2 * kt + 1][i], xy[1], 0, 0, 0);
        }
      }
      // this wave's two key tiles of the Gram products (B = the same operand: [K; Q] row n16 against keys)
#pragma unroll
      for (int kk = 0; kk < 2; ++kk) {
        const f32x4_t a4 = *reinterpret_cast<const f32x4_t*>(arow + (2 * wave + kk) * (ROWS + 4));
#pragma unroll
        for (int i = 0; i < 4; ++i) gr = __builtin_amdgcn_mfma_f32_16x16x4f32(a4[i], a4[i], gr, 0, 0, 0);
      }
      // partial Gram rows 0-15 (k_t or q_t against k_s, s < CT): lanes n16 < CT of every row group
      if (n16 < CT) {
#pragma unroll
        for (int i = 0; i < 4; ++i) gp_[wave][(4 * j4 + i) & (CT - 1)][(j4 >> 1) * CT + n16] = gr[i];
      }
      lds_barrier();
      // the burst's small matrices, by wave 0 (the others wait at the barrier below). gamma = 1, beta = 0 past nt.
      //   lane 8 t + s: A[t][s] = beta_t Gamma_t / Gamma_s (k_t . k_s) for s < t and Bm[t][s] = Gamma_t / Gamma_s
      //   (q_t . k_s) for s <= t, from the four waves' partial Gram sums; lanes 0-7: the factors Gamma_t D and c_t,
      //   then column t of T = (I + A)^-1 by forward substitution over A read back from LDS. Every operand is
      //   loaded before the arithmetic that uses it (no LDS round trip per term).
      if (wave == 0) {
        const int ln = lane;
        float g8[CT];
#pragma unroll
        for (int r = 0; r < CT; ++r) g8[r] = r < nt ? sdec_[r] : 1.0f;
        {
          const int t = ln >> 3, sc = ln & 7;
          float kk = 0.f, qk = 0.f;
#pragma unroll
          for (int w4 = 0; w4 < 4; ++w4) {
            kk += gp_[w4][t][sc];
            qk += gp_[w4][t][CT + sc];
          }
          float ratio = 1.0f;   // Gamma_t / Gamma_sc = product of gamma over (sc, t]
#pragma unroll
          for (int r = 1; r < CT; ++r) ratio *= (r > sc && r <= t) ? g8[r] : 1.0f;
          am_[t][sc] = sc < t && t < nt ? sbe_[t] * ratio * kk : 0.0f;
          bm_[t][sc] = sc <= t ? ratio * qk : 0.0f;
        }
        if (ln < CT) {
          float g_to_t = 1.0f, g_after = 1.0f, gcw = 1.0f;   // Gamma_t, Gamma_C / Gamma_t, Gamma_C
#pragma unroll
          for (int r = 0; r < CT; ++r) {
            g_to_t *= r <= ln ? g8[r] : 1.0f;
            g_after *= r > ln ? g8[r] : 1.0f;
            gcw *= g8[r];
          }
          fac_[0][ln] = g_to_t * D;
          fac_[1][ln] = D * gcw < 0x1p-40f ? g_after : 1.0f / (g_to_t * D);
        }
        // the lanes' A entries are read by other lanes of this wave: a wave-scope fence orders them
        __builtin_amdgcn_fence(__ATOMIC_SEQ_CST, "wavefront");
        if (ln < CT) {
          const int sc = ln;   // column of T: T[t][sc] = -sum_{sc <= r < t} A[t][r] T[r][sc], T[sc][sc] = 1
          float a[CT][CT];
#pragma unroll
          for (int t = 1; t < CT; ++t)
#pragma unroll
            for (int r = 0; r < t; ++r) a[t][r] = am_[t][r];
          float tc[CT];
#pragma unroll
          for (int t = 0; t < CT; ++t) {
            float acc = 0.f;
#pragma unroll
            for (int r = 0; r < t; ++r) acc = fmaf(r >= sc ? a[t][r] : 0.0f, tc[r], acc);
            tc[t] = t < sc ? 0.0f : t == sc ? 1.0f : -acc;
          }
#pragma unroll
          for (int t = 0; t < CT; ++t) tm_[t][sc] = tc[t];
        }
      }
      lds_barrier();
      float gc = 1.0f;   // Gamma_C, the same product in every thread
      for (int r = 0; r < CT; ++r) gc *= r < nt ? sdec_[r] : 1.0f;
      f32x4_t w[2];
#pragma unroll
      for (int ct = 0; ct < 2; ++ct) {
        // Every LDS operand below is read unconditionally from a clamped index and pinned there, and the lane
        // conditions select after: a read inside a conditional compiles to a branch with its own wait.
        // R = beta (V - Gamma D X) on rows 0-7 (lanes j4 < 2); zero elsewhere
        f32x4_t rr, oc;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int t = (4 * j4 + i) & (CT - 1);
          const int cc = cbase + 16 * ct;
          const float v = loaded_here(CONV ? bf2f(co_[CONV ? t : 0][CONV ? 2 * KD + cc : 0]) : bf2f(sv_[t][cc]));
          const float be = loaded_here(sbe_[t]), f0 = loaded_here(fac_[0][t]);
          const float r = be * (v - f0 * xy[ct][i]);
          rr[i] = (j4 < 2 && t < nt) ? r : 0.0f;
          oc[i] = j4 >= 2 ? f0 * xy[ct][i] : 0.0f;   // O's C input: Gamma D Y (rows 8-15)
        }
        float ta[2], ba[2];
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const float tv = loaded_here(tm_[n16 & (CT - 1)][tau(s2, j4)]);
          const float bv = loaded_here(bm_[n16 & (CT - 1)][tau(s2, j4)]);
          ta[s2] = n16 < CT ? tv : 0.0f;
          ba[s2] = n16 >= CT ? bv : 0.0f;
        }
        // V' = T R (rows 0-7)
        f32x4_t vp = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) vp = __builtin_amdgcn_mfma_f32_16x16x4f32(ta[s2], bop(rr, s2), vp, 0, 0, 0);
        // O = Gamma D Y + Bm V' (rows 8-15: the lanes holding Y)
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) oc = __builtin_amdgcn_mfma_f32_16x16x4f32(ba[s2], bop(vp, s2), oc, 0, 0, 0);
        // the burst's outputs (rows 8-15) -> so_, rounded to bf16 as the token path stores them. Rows at and past
        // nt hold padding tokens' outputs, which the epilogue reads but never stores.
        if (j4 >= 2) {
#pragma unroll
          for (int i = 0; i < 4; ++i) so_[4 * (j4 - 2) + i][cbase + 16 * ct] = rbf(oc[i]);
        }
        // W = c V' (rows 0-7) for the state update
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float f1 = loaded_here(fac_[1][(4 * j4 + i) & (CT - 1)]);
          w[ct][i] = j4 < 2 ? f1 * vp[i] : 0.0f;
        }
      }
      if (D * gc < 0x1p-40f) {   // uniform: fold D and the burst's decay into St before the update
        const float f = D * gc;
#pragma unroll
        for (int e = 0; e < 16; ++e) Sm[e] *= f;
        D = 1.0f;
      } else {
        D *= gc;
      }
      // S += K^T W: A = K^T (key 16 kt + n16, token tau), B = W
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const float b0 = bop(w[0], s2), b1 = bop(w[1], s2);
        const float* krow = &fk_[tau(s2, j4)][0][n16];
#pragma unroll
        for (int kt = 0; kt < KD / 16; ++kt) {
          const float a = krow[kt * (ROWS + 4)];
          Sm[2 * kt] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b0, Sm[2 * kt], 0, 0, 0);
          Sm[2 * kt + 1] = __builtin_amdgcn_mfma_f32_16x16x4f32(a, b1, Sm[2 * kt + 1], 0, 0, 0);
        }
      }
      if constexpr (GATED) {
        gated_epilogue(t0, nt);
      } else {
        __syncthreads();
        const int u = threadIdx.x >> 5, cc = (threadIdx.x & 31) * 4;
        if (u < nt) {
          const f32x4_t ob = *reinterpret_cast<const f32x4_t*>(&so_[u][cc]);
          const int64_t base = ((tok0 + t0 + u) * p.HV + hv) * VD + cc;
          const float o4[4] = {ob[0], ob[1], ob[2], ob[3]};
          store4_bf16(p.o + base, o4);
          if (p.sq != nullptr)
            *reinterpret_cast<float4*>(p.sq + base) = make_float4(ob[0] * ob[0], ob[1] * ob[1], ob[2] * ob[2],
                                                                  ob[3] * ob[3]);
        }
      }
      if (t0 + CT < ntok) {
        next_burst(t0);
        zero_pad(min(CT, ntok - t0 - CT));
      }
    }
    store_conv_history();
    zero_tail();
    const int st = tid_per_site();
    const int soff_st = (4 * ((st & 63) >> 4) * VD + (st >> 6) * TILE_V + (st & 15)) * (int)sizeof(ST);
#pragma unroll
    for (int kt = 0; kt < KD / 16; ++kt)
#pragma unroll
      for (int ct = 0; ct < 2; ++ct)
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int off = soff_st + (i * VD + 16 * ct) * (int)sizeof(ST);
          const float x = Sm[2 * kt + ct][i] * D;
          if constexpr (sizeof(ST) == 4)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(x), srs, off, kt * KT_BYTES, 2);   // nt
          else
            __builtin_amdgcn_raw_buffer_store_b16(f2h(x), srs, off, kt * KT_BYTES, 2);
        }
    return;
  }

  // Issue order: the first burst, the weights, then the state. Load counters retire in order, so staging the
  // burst (and the weights' copy to LDS) waits only for the loads issued before the state's and overlaps the
  // state's latency. Every load here is unconditional (the weight loads of surplus threads repeat the last
  // piece): a load under a branch makes the compiler wait for all outstanding loads where the paths join.
  if constexpr (CONV) fetch_first_conv();
  else fetch(0);
  u32x4 cwr[4], swr;
  const bool has_cw = CONV && threadIdx.x < CH3 / 8;   // 8 channels x 4 taps = 64 bytes per thread
  const bool has_sw = GATED && threadIdx.x < VD / 8;
  if constexpr (CONV) {
    const uint16_t* wsrc = p.conv_w + (int64_t)conv_ch(8 * min((int)threadIdx.x, CH3 / 8 - 1)) * CKS;
#pragma unroll
    for (int j = 0; j < 4; ++j) cwr[j] = *reinterpret_cast<const u32x4*>(wsrc + 8 * j);
  }
  if constexpr (GATED) swr = *reinterpret_cast<const u32x4*>(p.norm_w + 8 * min((int)threadIdx.x, VD / 8 - 1));
  __builtin_amdgcn_sched_barrier(0);   // keep the state loads last
#pragma unroll
  for (int j = 0; j < ROWS; ++j) StateIO<ST>::load(sp + j * VD, S[j]);
  if (has_cw) {
#pragma unroll
    for (int j = 0; j < 4; ++j) *reinterpret_cast<u32x4*>(&cw_[CONV ? 8 * threadIdx.x : 0][0] + 8 * j) = cwr[j];
  }
  if (has_sw) *reinterpret_cast<u32x4*>(&sw_[8 * threadIdx.x]) = swr;

  // The first burst is staged before the loop and each later one at the end of the previous iteration: a
  // staging at the top of the loop would merge the first iteration's wait with the back edge's and wait for
  // the state too.
  stage(min(CT, ntok), true);
  for (int t0 = 0; t0 < ntok; t0 += CT) {
    const int nt = min(CT, ntok - t0);
    if (t0 + CT < ntok) fetch(t0 + CT);
    __syncthreads();

    for (int tt = 0; tt < nt; ++tt) {
      float v[4];
      if constexpr (CONV) load4_bf16(&co_[CONV ? tt : 0][2 * KD + col], v);
      else load4_bf16(&sv_[tt][col], v);
      const float beta = sbe_[tt];
      float Dn = D * sdec_[tt];
      if (Dn < 0x1p-40f) {   // uniform over the workgroup (every lane has the same D and decay)
#pragma unroll
        for (int j = 0; j < ROWS; ++j)
#pragma unroll
          for (int i = 0; i < 4; ++i) S[j][i] *= Dn;
        Dn = 1.0f;
      }
      // S1 = exp(g) S_prev = Dn St;  v' = beta (v - S1^T k);  S2 = S1 + k v'^T = Dn (St + k (v' / Dn)^T);
      // o = S2^T q = Dn (St'^T q). q and k are read from LDS four rows at a time (147 VGPRs instead of 163).
      float kv[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < ROWS; j += 4) {
        const f32x4_t k4 = *reinterpret_cast<const f32x4_t*>(&fk_[tt][rg][j]);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int i = 0; i < 4; ++i) kv[i] += S[j + jj][i] * k4[jj];
      }
      const float rD = __builtin_amdgcn_rcpf(Dn);   // v_rcp_f32 (1 ulp): S2 is Dn * rD * (k v'^T), within 1e-7
      float w[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = beta * (v[i] - Dn * sum_rg(kv[i])) * rD;
      float o[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int j = 0; j < ROWS; j += 4) {
        const f32x4_t k4 = *reinterpret_cast<const f32x4_t*>(&fk_[tt][rg][j]);
        const f32x4_t q4 = *reinterpret_cast<const f32x4_t*>(&fq_[tt][rg][j]);
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            S[j + jj][i] += k4[jj] * w[i];
            o[i] += S[j + jj][i] * q4[jj];
          }
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) o[i] = sum_rg(o[i]) * Dn;
      D = Dn;

      const int64_t tok = tok0 + t0 + tt;
      if constexpr (!GATED) {
        if (rg == 0) {
          const int64_t base = (tok * p.HV + hv) * VD + col;
          store4_bf16(p.o + base, o);
          if (p.sq != nullptr) {
            float s4[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
              const float ob = rbf(o[i]);
              s4[i] = ob * ob;
            }
            *reinterpret_cast<float4*>(p.sq + base) = make_float4(s4[0], s4[1], s4[2], s4[3]);
          }
        }
      } else {
        if (rg == 0) {
          const f32x4_t ob = {rbf(o[0]), rbf(o[1]), rbf(o[2]), rbf(o[3])};
          *reinterpret_cast<f32x4_t*>(&so_[tt][col]) = ob;
        }
      }
    }

    if constexpr (GATED) gated_epilogue(t0, nt);
    if (t0 + CT < ntok) next_burst(t0);
  }

  store_conv_history();
  zero_tail();

#pragma unroll
  for (int j = 0; j < ROWS; ++j) {
#pragma unroll
    for (int i = 0; i < 4; ++i) S[j][i] *= D;
    StateIO<ST>::store(sp + j * VD, S[j]);
  }
}

int check_common(const GdnParams& p, int state_dtype, int n_rows, int K, int V) {
  if (n_rows < 0 || p.H <= 0 || p.HV <= 0 || p.L < 0 || p.state_rows <= 0 || p.mfma_min < 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  if (!p.qkv || !p.a || !p.b || !p.A_log || !p.dt_bias || !p.state || !p.slots || !p.lens) return HSG_ERR_ARG;
  if (p.offsets == nullptr && p.L <= 0) return HSG_ERR_ARG;
  if (K != KD || V != VD || p.HV % p.H != 0) return HSG_ERR_SHAPE;
  if (state_dtype != HSG_STATE_F32 && state_dtype != HSG_STATE_F16) return HSG_ERR_ARG;
  if (!aligned(p.qkv, 16) || p.qkv_stride % 8 || p.q_off % 8 || p.k_off % 8 || p.v_off % 8) return HSG_ERR_ALIGN;
  if (!aligned(p.state, 16)) return HSG_ERR_ALIGN;
  return 1;  // proceed
}

template <bool GATED, bool CONV = false>
int launch(const GdnParams& p, int state_dtype, int n_rows, void* stream) {
  const dim3 grid((unsigned)(n_rows * p.HV));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (state_dtype == HSG_STATE_F32)
    hipLaunchKernelGGL((gdn_step_kernel<float, GATED, CONV>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gdn_step_kernel<uint16_t, GATED, CONV>), grid, dim3(256), 0, s, p);
  return launch_status();
}

}  // namespace
}  // namespace hsg

using hsg::GdnParams;

extern "C" int hsg_gdn_slot_step(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off,
                                 int32_t v_off, const void* a, const void* b, int64_t ab_stride,
                                 const void* A_log, const void* dt_bias, void* state, int32_t state_dtype,
                                 int64_t state_rows, const int64_t* slots, const int64_t* lens,
                                 const int64_t* offsets, int32_t n_rows, int32_t L, int32_t H, int32_t HV,
                                 int32_t K, int32_t V, float scale, void* o, float* sq, int32_t burst_min,
                                 void* stream) {
  GdnParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qkv_stride = qkv_stride;
  p.q_off = q_off; p.k_off = k_off; p.v_off = v_off;
  p.a = static_cast<const uint16_t*>(a);
  p.b = static_cast<const uint16_t*>(b);
  p.ab_stride = ab_stride;
  p.A_log = static_cast<const uint16_t*>(A_log);
  p.dt_bias = static_cast<const uint16_t*>(dt_bias);
  p.state = state;
  p.state_rows = state_rows;
  p.slots = slots; p.lens = lens; p.offsets = offsets;
  p.L = L; p.H = H; p.HV = HV; p.scale = scale;
  p.o = static_cast<uint16_t*>(o);
  p.sq = sq;
  p.mfma_min = burst_min;
  const int rc = hsg::check_common(p, state_dtype, n_rows, K, V);
  if (rc <= 0) return rc;
  if (!o) return HSG_ERR_ARG;
  if (!hsg::aligned(o, 8) || (sq && !hsg::aligned(sq, 16))) return HSG_ERR_ALIGN;
  return hsg::launch<false>(p, state_dtype, n_rows, stream);
}

extern "C" int hsg_gdn_slot_step_gated(const void* qkv, int64_t qkv_stride, int32_t q_off, int32_t k_off,
                                       int32_t v_off, const void* a, const void* b, int64_t ab_stride,
                                       const void* A_log, const void* dt_bias, void* state,
                                       int32_t state_dtype, int64_t state_rows, const int64_t* slots,
                                       const int64_t* lens, const int64_t* offsets, int32_t n_rows, int32_t L,
                                       int32_t H, int32_t HV, int32_t K, int32_t V, float scale,
                                       const void* z, int64_t z_stride, const void* norm_w, float eps,
                                       void* out, int32_t skip_rows, int32_t skip_min_len, int32_t burst_min,
                                       void* stream) {
  GdnParams p{};
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qkv_stride = qkv_stride;
  p.q_off = q_off; p.k_off = k_off; p.v_off = v_off;
  p.a = static_cast<const uint16_t*>(a);
  p.b = static_cast<const uint16_t*>(b);
  p.ab_stride = ab_stride;
  p.A_log = static_cast<const uint16_t*>(A_log);
  p.dt_bias = static_cast<const uint16_t*>(dt_bias);
  p.state = state;
  p.state_rows = state_rows;
  p.slots = slots; p.lens = lens; p.offsets = offsets;
  p.L = L; p.H = H; p.HV = HV; p.scale = scale;
  p.z = static_cast<const uint16_t*>(z);
  p.z_stride = z_stride;
  p.norm_w = static_cast<const uint16_t*>(norm_w);
  p.eps = eps;
  p.out = static_cast<uint16_t*>(out);
  p.skip_rows = skip_rows;
  p.skip_min_len = skip_min_len;
  p.mfma_min = burst_min;
  const int rc = hsg::check_common(p, state_dtype, n_rows, K, V);
  if (rc <= 0) return rc;
  if (!z || !norm_w || !out || skip_rows < 0 || (skip_rows > 0 && skip_min_len < 1)) return HSG_ERR_ARG;
  if (!hsg::aligned(z, 16) || z_stride % 8 || !hsg::aligned(norm_w, 16) || !hsg::aligned(out, 8)) return HSG_ERR_ALIGN;
  return hsg::launch<true>(p, state_dtype, n_rows, stream);
}

extern "C" int hsg_gdn_conv_slot_step_gated(const void* proj, int64_t proj_stride, int32_t q_off, int32_t k_off,
                                            int32_t v_off, const void* conv_w, void* conv_pool, int32_t channels,
                                            const void* a, const void* b, int64_t ab_stride, const void* A_log,
                                            const void* dt_bias, void* state, int32_t state_dtype,
                                            int64_t state_rows, const int64_t* slots, const int64_t* lens,
                                            const int64_t* offsets, int32_t n_rows, int32_t H, int32_t HV,
                                            int32_t K, int32_t V, float scale, const void* z, int64_t z_stride,
                                            const void* norm_w, float eps, void* out, int32_t burst_min,
                                            void* stream) {
  GdnParams p{};
  p.qkv = static_cast<const uint16_t*>(proj);
  p.qkv_stride = proj_stride;
  p.q_off = q_off; p.k_off = k_off; p.v_off = v_off;
  p.a = static_cast<const uint16_t*>(a);
  p.b = static_cast<const uint16_t*>(b);
  p.ab_stride = ab_stride;
  p.A_log = static_cast<const uint16_t*>(A_log);
  p.dt_bias = static_cast<const uint16_t*>(dt_bias);
  p.state = state;
  p.state_rows = state_rows;
  p.slots = slots; p.lens = lens; p.offsets = offsets;
  p.L = 0; p.H = H; p.HV = HV; p.scale = scale;
  p.z = static_cast<const uint16_t*>(z);
  p.z_stride = z_stride;
  p.norm_w = static_cast<const uint16_t*>(norm_w);
  p.eps = eps;
  p.out = static_cast<uint16_t*>(out);
  p.conv_w = static_cast<const uint16_t*>(conv_w);
  p.conv_pool = static_cast<uint16_t*>(conv_pool);
  p.conv_C = channels;
  if (!offsets) return HSG_ERR_ARG;   // packed rows only
  p.mfma_min = burst_min;
  const int rc = hsg::check_common(p, state_dtype, n_rows, K, V);
  if (rc <= 0) return rc;
  if (!z || !norm_w || !out || !conv_w || !conv_pool) return HSG_ERR_ARG;
  // one value head per key head: every (row, head) workgroup owns its q / k conv channels and history
  if (HV != H) return HSG_ERR_SHAPE;
  if (channels <= 0 || q_off < 0 || k_off < 0 || v_off < 0 || q_off + H * K > channels || k_off + H * K > channels ||
      v_off + HV * V > channels || channels > proj_stride)
    return HSG_ERR_ARG;
  if (channels % 8 || !hsg::aligned(conv_w, 16) || !hsg::aligned(conv_pool, 16)) return HSG_ERR_ALIGN;
  if (!hsg::aligned(z, 16) || z_stride % 8 || !hsg::aligned(norm_w, 16) || !hsg::aligned(out, 8)) return HSG_ERR_ALIGN;
  return hsg::launch<true, true>(p, state_dtype, n_rows, stream);
}
