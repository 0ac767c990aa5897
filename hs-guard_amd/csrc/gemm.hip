// The step's projection GEMMs on hipBLASLt with a fixed algorithm per problem.
//
// torch.mm hands every call to hipBLASLt's first heuristic candidate. Faster solutions exist for the step's shapes
// (about 10-15 % on the mixed step's products), but a choice made by timing at start-up differs between processes,
// and solutions differ in accumulation order, so results would change from run to run. Here the solution is a
// caller-given hipBLASLt solution index, taken from a plan table generated once and committed
// (hs_guard/engine/gemm_plan.py); index -1 is the heuristic's first candidate. The reference's products are the
// nn.Linear layers of its backbone (src/hs_guard/engine/slot_engine_v8.py:52-53,63-65,72,78,89).
//
// Layout: D[M, N] = A[M, K] . W[N, K]^T, all row-major bf16 with row strides lda, ldw, ldd; fp32 accumulation. In
// hipBLASLt's column-major terms that is D^T (N x M) = op_T(W^T as K x N) . A^T (K x M).
#include <hipblaslt/hipblaslt-ext.hpp>
#include <hipblaslt/hipblaslt.h>

#include <map>
#include <mutex>
#include <tuple>
#include <vector>

#include "hsg_common.h"

namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t lw = nullptr, la = nullptr, ld = nullptr;
  hipblasLtMatmulAlgo_t algo{};
  size_t workspace = 0;
};

using PlanKey = std::tuple<int32_t, int32_t, int32_t, int64_t, int64_t, int64_t, int32_t>;

struct DeviceCtx {
  hipblasLtHandle_t handle = nullptr;
  std::map<PlanKey, Plan> plans;
};

constexpr int kMaxDevices = 64;
std::mutex ctx_mu;
DeviceCtx ctx[kMaxDevices];

// hipBLASLt status -> library code (HIP errors are positive, argument errors negative)
int blas_status(hipblasStatus_t s) { return s == HIPBLAS_STATUS_SUCCESS ? HSG_OK : HSG_ERR_BLAS; }

// the current device's context, its handle created on first use (call it outside graph capture first)
int device_ctx(DeviceCtx** out) {
  int dev = 0;
  const hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return (int)e;
  if (dev < 0 || dev >= kMaxDevices) return HSG_ERR_ARG;
  DeviceCtx& c = ctx[dev];
  if (c.handle == nullptr && hipblasLtCreate(&c.handle) != HIPBLAS_STATUS_SUCCESS) {
    c.handle = nullptr;
    return HSG_ERR_BLAS;
  }
  *out = &c;
  return HSG_OK;
}

void destroy_plan(Plan& p) {
  if (p.la) hipblasLtMatrixLayoutDestroy(p.la);
  if (p.lw) hipblasLtMatrixLayoutDestroy(p.lw);
  if (p.ld) hipblasLtMatrixLayoutDestroy(p.ld);
  if (p.desc) hipblasLtMatmulDescDestroy(p.desc);
  p = Plan{};
}

// descriptor and layouts of one problem (no algorithm yet)
int describe(int32_t M, int32_t N, int32_t K, int64_t lda, int64_t ldw, int64_t ldd, Plan& p) {
  const hipblasOperation_t op_w = HIPBLAS_OP_T, op_a = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &op_w, sizeof(op_w)) !=
          HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &op_a, sizeof(op_a)) !=
          HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.lw, HIP_R_16BF, K, N, ldw) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.la, HIP_R_16BF, K, M, lda) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.ld, HIP_R_16BF, N, M, ldd) != HIPBLAS_STATUS_SUCCESS) {
    destroy_plan(p);
    return HSG_ERR_BLAS;
  }
  return HSG_OK;
}

// up to `count` heuristic candidates for a described problem, in hipBLASLt's order, with workspace <= limit
int heuristic(DeviceCtx& c, Plan& p, size_t limit, int count, std::vector<hipblasLtMatmulHeuristicResult_t>& out) {
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return HSG_ERR_BLAS;
  uint64_t lim = limit;
  hipblasStatus_t s = hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &lim,
                                                            sizeof(lim));
  out.assign(count, hipblasLtMatmulHeuristicResult_t{});
  int found = 0;
  if (s == HIPBLAS_STATUS_SUCCESS)
    s = hipblasLtMatmulAlgoGetHeuristic(c.handle, p.desc, p.lw, p.la, p.ld, p.ld, pref, count, out.data(), &found);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (s != HIPBLAS_STATUS_SUCCESS || found <= 0) return HSG_ERR_BLAS;
  out.resize(found);
  return HSG_OK;
}

// heuristic candidates examined for solution -1
constexpr int kHeuristicCandidates = 16;

// the plan of a problem with the given solution (-1: the first heuristic candidate whose workspace fits `limit`),
// cached per device
int get_plan(DeviceCtx& c, int32_t M, int32_t N, int32_t K, int64_t lda, int64_t ldw, int64_t ldd, int32_t index,
             size_t limit, Plan** out) {
  const PlanKey key{M, N, K, lda, ldw, ldd, index};
  auto it = c.plans.find(key);
  if (it != c.plans.end()) {
    *out = &it->second;
    return HSG_OK;
  }
  Plan p;
  int rc = describe(M, N, K, lda, ldw, ldd, p);
  if (rc != HSG_OK) return rc;
  if (index < 0) {
    // the first candidate, in the heuristic's order, whose workspace fits: the hipBLASLt PyTorch ships returns
    // candidates beyond the preference's workspace limit (61 MiB against 32 at M = 11264, N = 7168, K = 1024)
    std::vector<hipblasLtMatmulHeuristicResult_t> res;
    rc = heuristic(c, p, limit, kHeuristicCandidates, res);
    if (rc != HSG_OK) {
      destroy_plan(p);
      return rc;
    }
    size_t pick = res.size();
    for (size_t i = 0; i < res.size() && pick == res.size(); ++i)
      if (res[i].workspaceSize <= limit) pick = i;
    if (pick == res.size()) {
      destroy_plan(p);
      return HSG_ERR_SHAPE;   // no candidate fits the caller's workspace
    }
    p.algo = res[pick].algo;
    p.workspace = res[pick].workspaceSize;
  } else {
    std::vector<int> idx{index};
    std::vector<hipblasLtMatmulHeuristicResult_t> res;
    const float alpha = 1.f, beta = 0.f;
    size_t ws = 0;
    // The library's C++ extension calls are bound from the hipBLASLt the process loaded (torch's bundled one, which
    // the plan table was generated with), not necessarily the release whose headers this file was compiled with;
    // their mangled signatures are the same in both. The round trip index -> algo -> index checks that the result
    // records were laid out as this build expects before one is used.
    if (hipblaslt_ext::getAlgosFromIndex(c.handle, idx, res) != HIPBLAS_STATUS_SUCCESS || res.size() != 1 ||
        hipblaslt_ext::getIndexFromAlgo(res[0].algo) != index ||
        hipblaslt_ext::matmulIsAlgoSupported(c.handle, p.desc, &alpha, p.lw, p.la, &beta, p.ld, p.ld, res[0].algo,
                                             ws) != HIPBLAS_STATUS_SUCCESS) {
      destroy_plan(p);
      return HSG_ERR_SHAPE;   // the solution does not exist in this hipBLASLt or does not support the problem
    }
    p.algo = res[0].algo;
    p.workspace = ws;
  }
  auto ins = c.plans.emplace(key, p);
  *out = &ins.first->second;
  return HSG_OK;
}

bool bad_problem(int32_t M, int32_t N, int32_t K, int64_t lda, int64_t ldw, int64_t ldd) {
  return M <= 0 || N <= 0 || K <= 0 || lda < K || ldw < K || ldd < N;
}

}  // namespace

extern "C" int hsg_gemm_bf16(const void* A, int64_t lda, const void* W, int64_t ldw, void* D, int64_t ldd,
                             int32_t M, int32_t N, int32_t K, int32_t algo_index, void* workspace,
                             size_t workspace_bytes, void* stream) {
  if (!A || !W || !D || bad_problem(M, N, K, lda, ldw, ldd) || algo_index < -1) return HSG_ERR_ARG;
  if (workspace_bytes > 0 && !workspace) return HSG_ERR_ARG;
  std::lock_guard<std::mutex> lock(ctx_mu);
  DeviceCtx* c = nullptr;
  int rc = device_ctx(&c);
  if (rc != HSG_OK) return rc;
  Plan* p = nullptr;
  rc = get_plan(*c, M, N, K, lda, ldw, ldd, algo_index, workspace_bytes, &p);
  if (rc != HSG_OK) return rc;
  if (p->workspace > workspace_bytes) return HSG_ERR_SHAPE;
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t s = hipblasLtMatmul(c->handle, p->desc, &alpha, W, p->lw, A, p->la, &beta, D, p->ld, D,
                                            p->ld, &p->algo, workspace, p->workspace,
                                            reinterpret_cast<hipStream_t>(stream));
  return blas_status(s);
}

extern "C" int hsg_gemm_candidates(int32_t M, int32_t N, int32_t K, int32_t* indices, size_t* workspace,
                                   int32_t max_count, size_t workspace_limit) {
  if (!indices || max_count <= 0 || bad_problem(M, N, K, K, K, N)) return -1;
  std::lock_guard<std::mutex> lock(ctx_mu);
  DeviceCtx* c = nullptr;
  if (device_ctx(&c) != HSG_OK) return -1;
  Plan p;
  if (describe(M, N, K, K, K, N, p) != HSG_OK) return -1;
  std::vector<hipblasLtMatmulHeuristicResult_t> res;
  const int rc = heuristic(*c, p, workspace_limit, max_count, res);
  destroy_plan(p);
  if (rc != HSG_OK) return -1;
  int n = 0;
  for (auto& r : res) {
    const int idx = hipblaslt_ext::getIndexFromAlgo(r.algo);
    if (idx < 0 || r.workspaceSize > workspace_limit) continue;   // the library does not always apply the limit
    indices[n] = idx;
    if (workspace) workspace[n] = r.workspaceSize;
    ++n;
  }
  return n;
}

namespace {

typedef __attribute__((ext_vector_type(2))) __bf16 bf16x2_t;

// Skinny products (M <= MM rows, the decode ticks): D[m, n] = sum_k A[m, k] W[n, k], bandwidth-bound on W. Each
// wave takes NC output columns (4 waves per workgroup); lane l takes the 8 elements 512 c + 8 l .. +7 of each
// 512-wide chunk c of K, so every load instruction of a wave reads 1 KB of one contiguous W row (a non-temporal
// load: the weights are read once per step, and keeping them out of the caches' way measured 4-7 % faster per
// product on MI355X). K runs in panels
// of CH chunks: the workgroup loads A's panel (MM rows x 512 CH) once into LDS while the waves' NC x CH W loads are
// in flight, then each wave takes A's pieces from LDS (conflict-free 16-byte reads, each used for NC columns),
// accumulates in fp32 on v_dot2_f32_bf16 (two products per instruction), reduces over the 64 lanes with the fixed
// DPP / permlane tree (so a result does not depend on timing), and rounds to bf16. Lane l's sum runs over its
// pieces in k order whatever MM, CH and NC are, so a row's result depends on its own inputs and K only.
// The operand A is staged in one of three modes:
//   PLAIN:   A as given;
//   SILU:    A is the MLP's gate|up projection (row m: gate in columns [0, K), up in [K, 2K)) and the operand is
//            bf16(bf16(silu(gate)) * up) with the rounding of hsg_silu_mul;
//   ADDNORM: K = 1024, A is the residual stream and the operand is the add + RMSNorm of hsg_add_rmsnorm
//            (bf16(A + mix), normalised, times w1), one wave per row in that kernel's lane layout (which is the
//            product's chunk layout at CH = 2) through the same row function; workgroup 0 writes the new residual
//            bf16(A + mix) to a separate buffer.
// Either way the result is bitwise that of the separate kernel followed by the PLAIN product.
enum SkinnyMode { PLAIN = 0, SILU = 1, ADDNORM = 2 };

struct SkinnyNorm {          // ADDNORM's extra operands, and an optional bias added before the output rounding
  const uint16_t* mix;
  int64_t ldm;
  const float* w1;
  float eps;
  uint16_t* hid_out;
  int64_t ldo;
  const uint16_t* bias;      // [N] bf16 or null
};

__device__ __forceinline__ float bf_at(uint32_t w, int hi) {
  return __uint_as_float(hi ? (w & 0xffff0000u) : (w << 16));
}

__device__ __forceinline__ hsg::u32x4 silu_mul8(hsg::u32x4 g, hsg::u32x4 u) {
  hsg::u32x4 y;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const uint32_t gw = g[j], uw = u[j];
    const float y0 = hsg::rbf(hsg::siluf_(bf_at(gw, 0))) * bf_at(uw, 0);
    const float y1 = hsg::rbf(hsg::siluf_(bf_at(gw, 1))) * bf_at(uw, 1);
    y[j] = (uint32_t)hsg::f2bf(y0) | ((uint32_t)hsg::f2bf(y1) << 16);
  }
  return y;
}

template <int MM, int CH, int NC, int MODE>
__global__ __launch_bounds__(256) void skinny_gemm_kernel(const uint16_t* A, int64_t lda, const uint16_t* W,
                                                          int64_t ldw, uint16_t* D, int64_t ldd, int M, int N, int K,
                                                          const SkinnyNorm nx) {
  static_assert(MODE != ADDNORM || CH == 2, "the add + RMSNorm staging covers one 1024-wide panel");
  constexpr int PIECES = 64 * CH;                    // 8-element pieces per A row per panel
  constexpr int STAGE = (MM * PIECES + 255) / 256;   // A pieces each thread stages per panel (PLAIN, SILU)
  constexpr int RW = (MM + 3) / 4;                   // rows each wave normalises (ADDNORM)
  __shared__ hsg::u32x4 a_lds[MM * PIECES];          // [MM][PIECES], MM * CH KiB
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int n0 = (blockIdx.x * 4 + wave) * NC;
  // a column past N is computed as column N - 1 and not stored, so every wave reaches the barriers
  const uint16_t* wrow[NC];
#pragma unroll
  for (int t = 0; t < NC; ++t) wrow[t] = W + (int64_t)min(n0 + t, N - 1) * ldw;
  // the bias, loaded up front (without one, W's first row stands in and is not used): a load under the output's
  // branch was compiled with a wait of its own at the end of the kernel
  const uint16_t* bsrc = nx.bias ? nx.bias : W;
  uint16_t bias_v[NC];
#pragma unroll
  for (int t = 0; t < NC; ++t) bias_v[t] = bsrc[min(n0 + t, N - 1)];
  float acc[NC][MM];
#pragma unroll
  for (int t = 0; t < NC; ++t)
#pragma unroll
    for (int m = 0; m < MM; ++m) acc[t][m] = 0.f;
  for (int kb = 0; kb < K; kb += 512 * CH) {
    // the panel's A loads first, then the W loads: waiting for A leaves W in flight
    hsg::u32x4 ap[MODE == ADDNORM ? 1 : STAGE];
    hsg::u32x4 hx[MODE == ADDNORM ? RW : 1][2], mx[MODE == ADDNORM ? RW : 1][2];
    hsg::f32x4_n wv[4];
    if constexpr (MODE == ADDNORM) {
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int mr = min(wave + 4 * r, M - 1);
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          hx[r][j] = *reinterpret_cast<const hsg::u32x4*>(A + (int64_t)mr * lda + 8 * lane + 512 * j);
          mx[r][j] = *reinterpret_cast<const hsg::u32x4*>(nx.mix + (int64_t)mr * nx.ldm + 8 * lane + 512 * j);
        }
      }
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        wv[2 * j] = *reinterpret_cast<const hsg::f32x4_n*>(nx.w1 + 8 * lane + 512 * j);
        wv[2 * j + 1] = *reinterpret_cast<const hsg::f32x4_n*>(nx.w1 + 8 * lane + 512 * j + 4);
      }
    } else {
#pragma unroll
      for (int i = 0; i < STAGE; ++i) {
        const int q = min(tid + 256 * i, MM * PIECES - 1);
        const int m = q / PIECES, p = q % PIECES;
        const uint16_t* apc = A + (int64_t)min(m, M - 1) * lda + min(kb + 8 * p, K - 8);
        if constexpr (MODE == SILU)
          ap[i] = silu_mul8(*reinterpret_cast<const hsg::u32x4*>(apc),
                            *reinterpret_cast<const hsg::u32x4*>(apc + K));
        else
          ap[i] = *reinterpret_cast<const hsg::u32x4*>(apc);
      }
    }
    hsg::u32x4 wv_[NC][CH];
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k0 = min(kb + 512 * c + 8 * lane, K - 8);   // clamped in bounds; pieces past K count as zero
#pragma unroll
      for (int t = 0; t < NC; ++t)
        wv_[t][c] = __builtin_nontemporal_load(reinterpret_cast<const hsg::u32x4*>(wrow[t] + k0));
    }
    __syncthreads();   // the previous panel's LDS reads are done
    if constexpr (MODE == ADDNORM) {
#pragma unroll
      for (int r = 0; r < RW; ++r) {
        const int m = wave + 4 * r;
        if (m < MM) {   // wave-uniform: the row function reduces over the whole wave
          hsg::u32x4 o[2];
          hsg::rmsnorm_row1024<true>(hx[r], mx[r], wv, nx.eps, o);
#pragma unroll
          for (int j = 0; j < 2; ++j) a_lds[m * PIECES + 64 * j + lane] = o[j];
          if (blockIdx.x == 0 && m < M) {
#pragma unroll
            for (int j = 0; j < 2; ++j)
              *reinterpret_cast<hsg::u32x4*>(nx.hid_out + (int64_t)m * nx.ldo + 8 * lane + 512 * j) = hx[r][j];
          }
        }
      }
    } else {
#pragma unroll
      for (int i = 0; i < STAGE; ++i)
        if (tid + 256 * i < MM * PIECES) a_lds[tid + 256 * i] = ap[i];
    }
    __syncthreads();
#pragma unroll
    for (int c = 0; c < CH; ++c) {
      const int k = kb + 512 * c + 8 * lane;
      const bool live = k < K;
#pragma unroll
      for (int m = 0; m < MM; ++m) {
        const hsg::u32x4 av = a_lds[m * PIECES + 64 * c + lane];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          // both operands through plain uint32_t values: a bit_cast of a vector element lvalue (wv_[t][c][j])
          // reads element 0 whatever j is
          const uint32_t a2 = live ? av[j] : 0u;
#pragma unroll
          for (int t = 0; t < NC; ++t) {
            const uint32_t w2 = live ? wv_[t][c][j] : 0u;
            acc[t][m] = __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a2),
                                                        __builtin_bit_cast(bf16x2_t, w2), acc[t][m], false);
          }
        }
      }
    }
  }
#pragma unroll
  for (int t = 0; t < NC; ++t) {
    float out = 0.f;
#pragma unroll
    for (int m = 0; m < MM; ++m) {
      const float s = hsg::wave_sum(acc[t][m]);
      if (lane == m) out = s;
    }
    if (n0 + t < N && lane < M) {
      if (nx.bias) out += hsg::bf2f(bias_v[t]);   // the Linear's bias in fp32, then one rounding
      D[(int64_t)lane * ldd + n0 + t] = hsg::f2bf(out);
    }
  }
}

// columns per wave: two where K is short (K <= 1024, the products of width 7168 and more), so each wave has 4 KB of
// W in flight and the grid fits the chip in one round; measured on MI355X against one and four per wave
template <int MM, int CH, int MODE>
void launch_skinny_nc(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, uint16_t* d, int64_t ldd,
                      int M, int N, int K, const SkinnyNorm& nx, hipStream_t st) {
  if (K <= 1024)
    hipLaunchKernelGGL((skinny_gemm_kernel<MM, CH, 2, MODE>), dim3((N + 7) / 8), dim3(256), 0, st, a, lda, w, ldw, d,
                       ldd, M, N, K, nx);
  else
    hipLaunchKernelGGL((skinny_gemm_kernel<MM, CH, 1, MODE>), dim3((N + 3) / 4), dim3(256), 0, st, a, lda, w, ldw, d,
                       ldd, M, N, K, nx);
}

template <int MM, int MODE>
void launch_skinny_k(const uint16_t* a, int64_t lda, const uint16_t* w, int64_t ldw, uint16_t* d, int64_t ldd, int M,
                     int N, int K, const SkinnyNorm& nx, hipStream_t st) {
  if (K <= 1024)
    launch_skinny_nc<MM, 2, MODE>(a, lda, w, ldw, d, ldd, M, N, K, nx, st);
  else if constexpr (MODE != ADDNORM) {
    if (K <= 2048)
      launch_skinny_nc<MM, 4, MODE>(a, lda, w, ldw, d, ldd, M, N, K, nx, st);
    else
      launch_skinny_nc<MM, 8, MODE>(a, lda, w, ldw, d, ldd, M, N, K, nx, st);
  }
}

template <int MODE>
int launch_skinny(const void* A, int64_t lda, const void* W, int64_t ldw, void* D, int64_t ldd, int M, int N, int K,
                  const SkinnyNorm& nx, void* stream) {
  using namespace hsg;
  if (!A || !W || !D || M <= 0 || N <= 0 || K <= 0 || lda < (MODE == SILU ? 2 : 1) * (int64_t)K || ldw < K ||
      ldd < N)
    return HSG_ERR_ARG;
  if (M > HSG_GEMM_SKINNY_M_MAX) return HSG_ERR_SHAPE;
  if (K % 8 || lda % 8 || ldw % 8 || !aligned(A, 16) || !aligned(W, 16) || !aligned(D, 2)) return HSG_ERR_ALIGN;
  hipStream_t st = reinterpret_cast<hipStream_t>(stream);
  const uint16_t* a = static_cast<const uint16_t*>(A);
  const uint16_t* w = static_cast<const uint16_t*>(W);
  uint16_t* d = static_cast<uint16_t*>(D);
  if (M == 1)
    launch_skinny_k<1, MODE>(a, lda, w, ldw, d, ldd, M, N, K, nx, st);
  else if (M == 2)
    launch_skinny_k<2, MODE>(a, lda, w, ldw, d, ldd, M, N, K, nx, st);
  else if (M <= 4)
    launch_skinny_k<4, MODE>(a, lda, w, ldw, d, ldd, M, N, K, nx, st);
  else
    launch_skinny_k<8, MODE>(a, lda, w, ldw, d, ldd, M, N, K, nx, st);
  return launch_status();
}

}  // namespace

extern "C" int hsg_gemm_bf16_skinny(const void* A, int64_t lda, const void* W, int64_t ldw, void* D, int64_t ldd,
                                    int32_t M, int32_t N, int32_t K, void* stream) {
  return launch_skinny<PLAIN>(A, lda, W, ldw, D, ldd, M, N, K, SkinnyNorm{}, stream);
}

extern "C" int hsg_gemm_bf16_skinny_silu(const void* gate_up, int64_t ld_gu, const void* W, int64_t ldw, void* D,
                                         int64_t ldd, int32_t M, int32_t N, int32_t K, void* stream) {
  return launch_skinny<SILU>(gate_up, ld_gu, W, ldw, D, ldd, M, N, K, SkinnyNorm{}, stream);
}

extern "C" int hsg_gemm_bf16_skinny_addnorm(const void* hidden, int64_t ldh, const void* mix, int64_t ldm,
                                            const float* w1, float eps, void* hidden_out, int64_t ldo, const void* W,
                                            int64_t ldw, void* D, int64_t ldd, int32_t M, int32_t N, int32_t K,
                                            const void* bias, void* stream) {
  using namespace hsg;
  if (!mix || !w1 || !hidden_out || hidden_out == hidden || ldm < K || ldo < K) return HSG_ERR_ARG;
  if (K != 1024) return HSG_ERR_SHAPE;
  if (ldm % 8 || ldo % 8 || !aligned(mix, 16) || !aligned(w1, 16) || !aligned(hidden_out, 16) ||
      (bias && !aligned(bias, 2)))
    return HSG_ERR_ALIGN;
  const SkinnyNorm nx{static_cast<const uint16_t*>(mix), ldm, w1, eps, static_cast<uint16_t*>(hidden_out), ldo,
                      static_cast<const uint16_t*>(bias)};
  return launch_skinny<ADDNORM>(hidden, ldh, W, ldw, D, ldd, M, N, K, nx, stream);
}

extern "C" int hsg_gemm_blas_version(void) {
  std::lock_guard<std::mutex> lock(ctx_mu);
  DeviceCtx* c = nullptr;
  if (device_ctx(&c) != HSG_OK) return -1;
  int v = 0;
  return hipblasLtGetVersion(c->handle, &v) == HIPBLAS_STATUS_SUCCESS ? v : -1;
}
