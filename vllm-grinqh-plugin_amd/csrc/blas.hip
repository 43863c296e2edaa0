// Library GEMM of a large dense prefill: Y[M][N] = X[M][K] @ Wt[N][K]^T
// (+ bias), fp32 accumulation, through hipBLASLt.
//
// Replaces the `X @ Wd` of grinqh_prefill_gemm_compiled (grinqh/kernel.py:587)
// and its bias add (:707-708).  The weight comes from dequant.hip, stored
// K-contiguous: in hipBLASLt's column-major terms D (N x M, ld N) =
// op(A) * B with A = Wt (K x N, ld K, transposed) and B = X (K x M, ld ldx),
// the "TN" form, which ran 10-40 % faster here than the K x N weight.
//
// The bias goes through the GEMM's bias epilogue: y = RNE(acc + bias), one
// rounding, where the reference rounds twice (RNE(RNE(acc) + bias)); the two
// differ by at most one unit in the last place of y.
//
// One hipBLASLt handle per device (created on first use, kept for the
// process); the descriptors and the chosen algorithm of each shape are
// cached per thread, so a call after the first only sets the bias pointer and
// enqueues the GEMM.
#include <hipblaslt/hipblaslt.h>

#include <mutex>
#include <vector>

#include "grinqh_launch.h"

namespace grinqh {

namespace {

constexpr int kMaxDevices = 64;

hipblasLtHandle_t handle_for_device(int dev) {
  static std::mutex mu;
  static hipblasLtHandle_t handles[kMaxDevices] = {};
  std::lock_guard<std::mutex> lock(mu);
  if (handles[dev] == nullptr) {
    hipblasLtHandle_t h = nullptr;
    if (hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) return nullptr;
    handles[dev] = h;
  }
  return handles[dev];
}

struct GemmShape {
  int dev;
  int64_t M, N, K, ldx;
  int dtype;
  bool bias;
  size_t ws_bytes;
  bool operator==(const GemmShape& o) const {
    return dev == o.dev && M == o.M && N == o.N && K == o.K && ldx == o.ldx && dtype == o.dtype &&
           bias == o.bias && ws_bytes == o.ws_bytes;
  }
};

struct GemmPlan {
  GemmShape shape;
  hipblasLtMatmulDesc_t desc;
  hipblasLtMatrixLayout_t a, b, d;
  hipblasLtMatmulAlgo_t algo;
  size_t algo_ws;
};

// Builds the descriptors of one shape and asks the heuristic for its best
// algorithm within ws_bytes of workspace.
bool make_plan(const GemmShape& s, GemmPlan& pl) {
  const hipDataType dt = s.dtype == GRINQH_DTYPE_BF16 ? HIP_R_16BF : HIP_R_16F;
  pl.shape = s;
  if (hipblasLtMatmulDescCreate(&pl.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT));
  hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN));
  if (s.bias) {
    const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bdt = dt;
    hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
    hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bdt, sizeof(bdt));
  }
  if (hipblasLtMatrixLayoutCreate(&pl.a, dt, (uint64_t)s.K, (uint64_t)s.N, s.K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&pl.b, dt, (uint64_t)s.K, (uint64_t)s.M, s.ldx) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&pl.d, dt, (uint64_t)s.N, (uint64_t)s.M, s.N) != HIPBLAS_STATUS_SUCCESS)
    return false;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
  const uint64_t ws = s.ws_bytes;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws));
  hipblasLtMatmulHeuristicResult_t res[1];
  int found = 0;
  const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(handle_for_device(s.dev), pl.desc, pl.a, pl.b, pl.d,
                                                             pl.d, pref, 1, res, &found);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS || found < 1 || res[0].workspaceSize > s.ws_bytes) return false;
  pl.algo = res[0].algo;
  pl.algo_ws = res[0].workspaceSize;
  return true;
}

}  // namespace

int gemm_x_wt(const uint16_t* x, int64_t ldx, const uint16_t* wt, const uint16_t* bias, uint16_t* y, int64_t M,
              int64_t N, int64_t K, int dtype, void* ws, size_t ws_bytes, hipStream_t st) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GRINQH_ERR_HIP;
  hipblasLtHandle_t h = handle_for_device(dev);
  if (h == nullptr) return GRINQH_ERR_HIP;
  thread_local std::vector<GemmPlan> plans;
  const GemmShape key{dev, M, N, K, ldx, dtype, bias != nullptr, ws_bytes};
  GemmPlan* pl = nullptr;
  for (GemmPlan& q : plans)
    if (q.shape == key) pl = &q;
  if (pl == nullptr) {
    GemmPlan q{};
    if (!make_plan(key, q)) return GRINQH_ERR_HIP;
    plans.push_back(q);
    pl = &plans.back();
  }
  if (bias != nullptr) {
    const void* bp = bias;
    hipblasLtMatmulDescSetAttribute(pl->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp));
  }
  const float alpha = 1.f, beta = 0.f;
  const hipblasStatus_t s = hipblasLtMatmul(h, pl->desc, &alpha, wt, pl->a, x, pl->b, &beta, y, pl->d, y, pl->d,
                                            &pl->algo, ws, pl->algo_ws, st);
  return s == HIPBLAS_STATUS_SUCCESS ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
