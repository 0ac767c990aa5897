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
// read with ordinary loads and written back with nontemporal stores (it is touched once per tick, so the
// write should not displace cached weights and activations); measured on MI355X this pairing streams
// faster than nontemporal loads (6.0 vs 5.4 TB/s at 352 x 16).
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
};

template <typename ST>
struct StateIO;

typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

template <>
struct StateIO<float> {
  static __device__ __forceinline__ void load(const float* p, float* v) {
    const f32x4_t x = *reinterpret_cast<const f32x4_t*>(p);
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
    const u32x2_t w = *reinterpret_cast<const u32x2_t*>(p);
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

template <typename ST, bool GATED>
__global__ __launch_bounds__(256) void gdn_step_kernel(const GdnParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int c = lane & 7;
  const int rg = lane >> 3;
  const int n = blockIdx.x / p.HV;
  const int hv = blockIdx.x - n * p.HV;
  const int h = hv / (p.HV / p.H);
  const int64_t slot = p.slots[n];
  int ntok = (int)p.lens[n];
  const bool padded = p.offsets == nullptr;
  if (slot < 0 || slot >= p.state_rows || ntok < 0) ntok = 0;
  if (padded && ntok > p.L) ntok = p.L;  // a row never reads past its L padded positions
  if (!padded && n < p.skip_rows && ntok >= p.skip_min_len) ntok = 0;   // routed to the chunk kernels
  const int64_t tok0 = padded ? (int64_t)n * p.L : p.offsets[n];
  const int col = wave * TILE_V + c * 4;

  // The registers hold St with S = D * St: the per-token decay multiplies the scalar D instead of all 64
  // registers; D is folded back into St before 1 / D could overflow and when the state is stored.
  float S[ROWS][4];
  float D = 1.0f;
  ST* sp = reinterpret_cast<ST*>(p.state) + ((slot * p.HV + hv) * KD + rg * ROWS) * (int64_t)VD + col;
  if (ntok > 0) {
#pragma unroll
    for (int j = 0; j < ROWS; ++j) StateIO<ST>::load(sp + j * VD, S[j]);
  }
  const float A = expf(bf2f(p.A_log[hv]));
  const float dt = bf2f(p.dt_bias[hv]);
  // per burst: normalised q (times scale) and k in fp32, one 16-row piece per lane group (stride 20 floats, so
  // the 8 pieces a wave reads at once fall on distinct banks); raw v and z; exp(g) and beta per token
  __shared__ __align__(16) float fq_[CT][KD / ROWS][ROWS + 4];
  __shared__ __align__(16) float fk_[CT][KD / ROWS][ROWS + 4];
  __shared__ __align__(16) uint16_t sv_[CT][VD];
  __shared__ __align__(16) uint16_t sz_[GATED ? CT : 1][VD];
  __shared__ __align__(16) float so_[GATED ? CT : 1][VD];   // bf16-rounded o of the burst, for the gated norm
  __shared__ float sdec_[CT], sbe_[CT];
  constexpr int SEGS = GATED ? 64 : 48;   // 16-byte segments per token: q, k, v (, z)
  constexpr int PF = (CT * SEGS + 255) / 256;   // segments per thread per burst (the last partly idle)
  // gated-norm weights staged in LDS once (read per token from global memory they were reloaded after every
  // output store, since `out` may alias them: one global round trip per token)
  __shared__ __align__(16) uint16_t sw_[GATED ? VD : 1];
  if (GATED && threadIdx.x < VD / 8)
    *reinterpret_cast<u32x4*>(&sw_[8 * threadIdx.x]) = *reinterpret_cast<const u32x4*>(p.norm_w + 8 * threadIdx.x);

  // The tokens of a row go through LDS in bursts of CT; the next burst is loaded into registers while the
  // current one is processed. Segment e = threadIdx.x + 256 i of a burst is token e / SEGS, piece e % SEGS
  // (pieces 16j .. 16j+15 are q, k, v, z for j = 0..3: an aligned group of 16 lanes holds one whole vector);
  // positions past the row's end re-read its last token (never stored to LDS).
  u32x4 pf[PF];
  uint16_t pa = 0, pb = 0;
  auto fetch = [&](int t) {
    const int last = ntok - 1 - t;
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int e = threadIdx.x + 256 * i;
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
    const int64_t tok = tok0 + t + min((int)threadIdx.x, last);
    pa = p.a[tok * p.ab_stride + hv];
    pb = p.b[tok * p.ab_stride + hv];
  };
  // prefetched burst -> LDS: q <- q / sqrt(|q|^2 + 1e-6) * scale and k <- k / sqrt(|k|^2 + 1e-6) once per token
  // (|x|^2 summed over the 16 lanes holding the vector), v and z as loaded, exp(g) and beta by thread u
  auto stage = [&](int nt) {
#pragma unroll
    for (int i = 0; i < PF; ++i) {
      const int e = threadIdx.x + 256 * i;
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
    if (threadIdx.x < nt) {
      const float x = bf2f(pa) + dt;
      const float g = -A * (x > 20.0f ? x : logf(1.0f + expf(x)));
      sdec_[threadIdx.x] = expf(g);
      sbe_[threadIdx.x] = sigmoidf_(bf2f(pb));
    }
  };
  if (ntok > 0) fetch(0);

  for (int t0 = 0; t0 < ntok; t0 += CT) {
    const int nt = min(CT, ntok - t0);
    __syncthreads();   // every read of the previous burst's LDS is done
    stage(nt);
    if (t0 + CT < ntok) fetch(t0 + CT);
    __syncthreads();

    for (int tt = 0; tt < nt; ++tt) {
      float v[4];
      load4_bf16(&sv_[tt][col], v);
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
          *reinterpret_cast<f32x4_t*>(&so_[GATED ? tt : 0][col]) = ob;
        }
      }
    }

    if constexpr (GATED) {
      // gated RMSNorm of the burst: 32 threads per token, 4 value columns each
      __syncthreads();
      const int u = threadIdx.x >> 5;
      const int cc = (threadIdx.x & 31) * 4;
      const f32x4_t ob = *reinterpret_cast<const f32x4_t*>(&so_[GATED ? u : 0][cc]);
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
    }
  }

  if (padded && rg == 0) {
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
  }

  if (ntok > 0) {
#pragma unroll
    for (int j = 0; j < ROWS; ++j) {
#pragma unroll
      for (int i = 0; i < 4; ++i) S[j][i] *= D;
      StateIO<ST>::store(sp + j * VD, S[j]);
    }
  }
}

int check_common(const GdnParams& p, int state_dtype, int n_rows, int K, int V) {
  if (n_rows < 0 || p.H <= 0 || p.HV <= 0 || p.L < 0 || p.state_rows <= 0) return HSG_ERR_ARG;
  if (n_rows == 0) return HSG_OK;
  if (!p.qkv || !p.a || !p.b || !p.A_log || !p.dt_bias || !p.state || !p.slots || !p.lens) return HSG_ERR_ARG;
  if (p.offsets == nullptr && p.L <= 0) return HSG_ERR_ARG;
  if (K != KD || V != VD || p.HV % p.H != 0) return HSG_ERR_SHAPE;
  if (state_dtype != HSG_STATE_F32 && state_dtype != HSG_STATE_F16) return HSG_ERR_ARG;
  if (!aligned(p.qkv, 16) || p.qkv_stride % 8 || p.q_off % 8 || p.k_off % 8 || p.v_off % 8) return HSG_ERR_ALIGN;
  if (!aligned(p.state, 16)) return HSG_ERR_ALIGN;
  return 1;  // proceed
}

template <bool GATED>
int launch(const GdnParams& p, int state_dtype, int n_rows, void* stream) {
  const dim3 grid((unsigned)(n_rows * p.HV));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (state_dtype == HSG_STATE_F32)
    hipLaunchKernelGGL((gdn_step_kernel<float, GATED>), grid, dim3(256), 0, s, p);
  else
    hipLaunchKernelGGL((gdn_step_kernel<uint16_t, GATED>), grid, dim3(256), 0, s, p);
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
                                 int32_t K, int32_t V, float scale, void* o, float* sq, void* stream) {
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
                                       void* out, int32_t skip_rows, int32_t skip_min_len, void* stream) {
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
  const int rc = hsg::check_common(p, state_dtype, n_rows, K, V);
  if (rc <= 0) return rc;
  if (!z || !norm_w || !out || skip_rows < 0 || (skip_rows > 0 && skip_min_len < 1)) return HSG_ERR_ARG;
  if (!hsg::aligned(z, 16) || z_stride % 8 || !hsg::aligned(norm_w, 16) || !hsg::aligned(out, 8)) return HSG_ERR_ALIGN;
  return hsg::launch<true>(p, state_dtype, n_rows, stream);
}
