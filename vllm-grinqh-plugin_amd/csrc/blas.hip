// Library GEMM of a large dense prefill: Y[M][N] = X[M][K] @ Wt[N][K]^T
// (+ bias), fp32 accumulation, through hipBLASLt.
//
// Replaces the `X @ Wd` of grinqh_prefill_gemm_compiled (grinqh/kernel.py:587)
// and its bias add (:707-708).  The weight comes from dequant.hip, stored
// K-contiguous: in hipBLASLt's column-major terms D (N x M, ld N) =
// op(A) * B with A = Wt (K x N, ld K, transposed) and B = X (K x M, ld ldx),
// the "TN" form, which ran 10-55 % faster here than the K x N weight.
//
// The product calls it without bias and adds the bias in a pass of its own
// (launch_add_bias_rows), so that y = RNE(RNE(acc) + bias) rounds twice as
// the reference's matmul followed by y.add_(bias) does; the GEMM's bias
// epilogue would round acc + bias once.
//
// One hipBLASLt handle per device (created on first use, kept for the
// process); the descriptors and the chosen algorithm of each shape are
// cached per thread, so a call after the first only sets the bias pointer and
// enqueues the GEMM.  The first call of a size class (M rounded up to a power
// of two) times the heuristic's candidates in the product's own sequence
// (fastest_candidate) and keeps the fastest: gate_up at 2048 rows 465 -> 428
// us for the whole product, gate_up and down at 8192 rows ~20 % faster, the
// other Llama-3-8B shapes unchanged.  The summation order of the GEMM
// depends on the algorithm, so a timed choice trades bit-for-bit
// reproducibility across processes for speed; GRINQH_GEMM_TUNE=0 (read once)
// keeps the heuristic's first candidate instead and times nothing.
//
// Only algorithms that use no workspace are taken.  The stream-K algorithms
// the heuristic prefers for the large shapes use one, and a graded gate_up
// product at 2048 rows captured in a HIP graph gave a wrong result on a
// replay after the first with them; the algorithms without workspace ran at
// the same speed (within 2 %) on the Llama-3-8B shapes at 512-8192 rows.
#include <hipblaslt/hipblaslt.h>

#include <cstdio>
#include <cstdlib>
#include <cstring>
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
  bool alpha_vector;  // per-output-column alpha read from device memory
  bool operator==(const GemmShape& o) const {
    return dev == o.dev && M == o.M && N == o.N && K == o.K && ldx == o.ldx && dtype == o.dtype &&
           bias == o.bias && alpha_vector == o.alpha_vector;
  }
};

struct GemmPlan {
  GemmShape shape;
  hipblasLtMatmulDesc_t desc;
  hipblasLtMatrixLayout_t a, b, d;
  hipblasLtMatmulAlgo_t algo;
};

// A failure of the library is reported on stderr with its status (the C ABI
// returns GRINQH_ERR_HIP): which step failed is otherwise not visible.
bool blas_failed(const char* what, int status, const GemmShape& s) {
  std::fprintf(stderr, "grinqh: hipBLASLt %s failed (status %d) for M=%lld N=%lld K=%lld ldx=%lld dtype=%d\n", what,
               status, (long long)s.M, (long long)s.N, (long long)s.K, (long long)s.ldx, s.dtype);
  return false;
}

// Size class of a timed algorithm choice.
struct TuneKey {
  int dev;
  int64_t m_bucket, N, K;
  int dtype;
  bool bias, alpha_vector;
  bool operator==(const TuneKey& o) const {
    return dev == o.dev && m_bucket == o.m_bucket && N == o.N && K == o.K && dtype == o.dtype && bias == o.bias &&
           alpha_vector == o.alpha_vector;
  }
};

// Operands of the call that creates a plan, for timing its candidates.
struct GemmCall {
  const void *wt, *x, *alpha, *beta;
  void* y;
  const void* bias;
  hipStream_t stream;
  const GemmPrelude* prelude;  // work that precedes the GEMM in the product (or nullptr)
};

// Times the candidate algorithms on the call's own operands, each run after
// the work that precedes the GEMM in the product (the weight's
// dequantization pass, which rewrites the weight operand and leaves the
// caches as the product does).  A warm-up run of each, then kRounds rounds
// that run every candidate in turn (so that clock and cache drift hit all
// alike), kRuns times back to back with events around each GEMM and one host
// wait per candidate and round (a host wait after every GEMM let the GPU idle
// between runs, and the timings then ranked some algorithms wrongly); each
// candidate keeps its fastest run.  Candidate 0 (the heuristic's first
// choice) is kept unless another is faster by more than kSwitchMargin.  The
// runs go to a private stream that first waits for the caller's stream, so
// every operand is complete and no work still pending there sees its memory
// change; the call itself writes y again afterwards.  Any failure keeps
// candidate 0.
int fastest_candidate(const GemmPlan& pl, const hipblasLtMatmulAlgo_t* algos, int n, const GemmCall& c) {
  constexpr int kRounds = 3, kRuns = 3;
  constexpr float kSwitchMargin = 0.05f;
  if (n < 2) return 0;
  hipStream_t ts = nullptr;
  hipEvent_t ready = nullptr, ev[2 * kRuns] = {};
  float best_ms[16];
  for (int i = 0; i < n; ++i) best_ms[i] = -1.f;  // not timed (or failed)
  bool ok = hipStreamCreateWithFlags(&ts, hipStreamNonBlocking) == hipSuccess &&
            hipEventCreateWithFlags(&ready, hipEventDisableTiming) == hipSuccess;
  for (hipEvent_t& e : ev) ok = ok && hipEventCreate(&e) == hipSuccess;
  ok = ok && hipEventRecord(ready, c.stream) == hipSuccess && hipStreamWaitEvent(ts, ready, 0) == hipSuccess;
  hipblasLtHandle_t h = handle_for_device(pl.shape.dev);
  bool runs[16];
  auto run = [&](int i) {
    return hipblasLtMatmul(h, pl.desc, c.alpha, c.wt, pl.a, c.x, pl.b, c.beta, c.y, pl.d, c.y, pl.d, &algos[i],
                           nullptr, 0, ts) == HIPBLAS_STATUS_SUCCESS;
  };
  auto prelude = [&] { return c.prelude == nullptr || (*c.prelude)(ts) == GRINQH_OK; };
  for (int i = 0; ok && i < n; ++i) runs[i] = run(i);  // warm-up (also loads each kernel)
  ok = ok && hipStreamSynchronize(ts) == hipSuccess;
  for (int round = 0; ok && round < kRounds; ++round)
    for (int i = 0; ok && i < n; ++i) {
      if (!runs[i]) continue;
      for (int r = 0; ok && r < kRuns; ++r)
        ok = prelude() && hipEventRecord(ev[2 * r], ts) == hipSuccess && run(i) &&
             hipEventRecord(ev[2 * r + 1], ts) == hipSuccess;
      ok = ok && hipEventSynchronize(ev[2 * kRuns - 1]) == hipSuccess;
      for (int r = 0; ok && r < kRuns; ++r) {
        float ms = 0.f;
        ok = hipEventElapsedTime(&ms, ev[2 * r], ev[2 * r + 1]) == hipSuccess;
        if (ok && (best_ms[i] < 0.f || ms < best_ms[i])) best_ms[i] = ms;
      }
    }
  int best = 0;
  if (ok && best_ms[0] > 0.f)
    for (int i = 1; i < n; ++i)
      if (best_ms[i] > 0.f && best_ms[i] < (1.f - kSwitchMargin) * best_ms[0] &&
          (best == 0 || best_ms[i] < best_ms[best]))
        best = i;
  if (ts != nullptr) {
    (void)hipStreamSynchronize(ts);
    (void)hipStreamDestroy(ts);
  }
  if (ready != nullptr) (void)hipEventDestroy(ready);
  for (hipEvent_t e : ev)
    if (e != nullptr) (void)hipEventDestroy(e);
  (void)hipGetLastError();
  return ok ? best : 0;
}

// The descriptors of one shape (bias_ptr: the bias epilogue's pointer, or
// nullptr when the shape has none).
bool build_descriptors(const GemmShape& s, GemmPlan& pl, const void* bias_ptr) {
  const hipDataType dt = s.dtype == GRINQH_DTYPE_BF16 ? HIP_R_16BF : HIP_R_16F;
  pl.shape = s;
  if (hipblasLtMatmulDescCreate(&pl.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS)
    return blas_failed("matmul descriptor", -1, s);
  const int32_t opT = HIPBLAS_OP_T, opN = HIPBLAS_OP_N;
  if (hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &opT, sizeof(opT)) !=
          HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &opN, sizeof(opN)) !=
          HIPBLAS_STATUS_SUCCESS)
    return blas_failed("transpose attributes", -1, s);
  if (s.alpha_vector) {  // alpha: device vector over the rows of D (the output columns), beta: host
    const int32_t mode = HIPBLASLT_POINTER_MODE_ALPHA_DEVICE_VECTOR_BETA_HOST;
    if (hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_POINTER_MODE, &mode, sizeof(mode)) !=
        HIPBLAS_STATUS_SUCCESS)
      return blas_failed("pointer mode attribute", -1, s);
  }
  if (s.bias) {
    const uint32_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const int32_t bdt = dt;
    if (hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bdt, sizeof(bdt)) !=
            HIPBLAS_STATUS_SUCCESS ||
        hipblasLtMatmulDescSetAttribute(pl.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias_ptr,
                                        sizeof(bias_ptr)) != HIPBLAS_STATUS_SUCCESS)
      return blas_failed("bias epilogue attributes", -1, s);
  }
  if (hipblasLtMatrixLayoutCreate(&pl.a, dt, (uint64_t)s.K, (uint64_t)s.N, s.K) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&pl.b, dt, (uint64_t)s.K, (uint64_t)s.M, s.ldx) != HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&pl.d, dt, (uint64_t)s.N, (uint64_t)s.M, s.N) != HIPBLAS_STATUS_SUCCESS)
    return blas_failed("matrix layout", -1, s);
  return true;
}

constexpr int kCandidates = 16;

// The heuristic's candidates for a described shape that need no workspace,
// in its order of preference: their count (0 if it offered none), or -1 if
// the query failed.  The heuristic does not always honour the workspace limit
// of the preference (Llama-3-70B qkv at 4096 rows: its first choice asked for
// 57 MiB of 32), so candidates that ask for workspace are dropped.
int workspace_free_candidates(const GemmPlan& pl, hipblasLtMatmulAlgo_t* algos) {
  const GemmShape& s = pl.shape;
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) {
    blas_failed("preference", -1, s);
    return -1;
  }
  const uint64_t ws = 0;
  if (hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &ws, sizeof(ws)) !=
      HIPBLAS_STATUS_SUCCESS) {
    hipblasLtMatmulPreferenceDestroy(pref);
    blas_failed("workspace preference", -1, s);
    return -1;
  }
  hipblasLtMatmulHeuristicResult_t res[kCandidates];
  int found = 0;
  const hipblasStatus_t st = hipblasLtMatmulAlgoGetHeuristic(handle_for_device(s.dev), pl.desc, pl.a, pl.b, pl.d,
                                                             pl.d, pref, kCandidates, res, &found);
  hipblasLtMatmulPreferenceDestroy(pref);
  if (st != HIPBLAS_STATUS_SUCCESS) {
    blas_failed("heuristic", (int)st, s);
    return -1;
  }
  int n = 0;
  for (int i = 0; i < found && i < kCandidates; ++i)
    if (res[i].state == HIPBLAS_STATUS_SUCCESS && res[i].workspaceSize == 0) algos[n++] = res[i].algo;
  return n;
}

// Builds the descriptors of one shape and takes, among the heuristic's
// candidates that need no workspace, the fastest on the creating call's
// operands (the heuristic's first choice ran the Llama-3-8B qkv, o_proj and
// down GEMMs at 0.9-1.1 PFLOP/s against 1.3 for gate_up).  While the caller's
// stream is being captured into a graph no candidate is run: the heuristic's
// first is taken (warm-up calls before the capture create the plans that are
// timed).
bool make_plan(const GemmShape& s, GemmPlan& pl, const GemmCall& call) {
  if (!build_descriptors(s, pl, call.bias)) return false;
  constexpr int kTimedCandidates = 8;
  hipblasLtMatmulAlgo_t algos[kCandidates];
  const int n = workspace_free_candidates(pl, algos);
  if (n < 0) return false;
  if (n == 0) return blas_failed("heuristic (no candidate without workspace)", -3, s);
  // The timed choice is kept per size class: M rounded up to a power of two
  // (with N, K, dtype and epilogue).  Another M of the class takes the same
  // algorithm when its own candidate list holds it, else its first candidate,
  // so that a new batch size does not time the candidates again.
  int64_t mb = 1;
  while (mb < s.M) mb <<= 1;
  const TuneKey tk{s.dev, mb, s.N, s.K, s.dtype, s.bias, s.alpha_vector};
  thread_local std::vector<std::pair<TuneKey, hipblasLtMatmulAlgo_t>> tuned;
  for (const auto& e : tuned) {
    if (!(e.first == tk)) continue;
    pl.algo = algos[0];
    for (int i = 0; i < n; ++i)
      if (std::memcmp(algos[i].data, e.second.data, sizeof(e.second.data)) == 0) pl.algo = algos[i];
    return true;
  }
  static const bool tune = [] {
    const char* v = std::getenv("GRINQH_GEMM_TUNE");
    return v == nullptr || std::strcmp(v, "0") != 0;
  }();
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  if (hipStreamIsCapturing(call.stream, &cap) != hipSuccess) cap = hipStreamCaptureStatusActive;
  if (!tune || cap != hipStreamCaptureStatusNone) {  // nothing is timed during a capture (nor remembered)
    pl.algo = algos[0];
    return true;
  }
  pl.algo = algos[fastest_candidate(pl, algos, n < kTimedCandidates ? n : kTimedCandidates, call)];
  tuned.emplace_back(tk, pl.algo);
  return true;
}

// Releases the descriptors of a plan that could not be completed.
void destroy_plan(GemmPlan& pl) {
  if (pl.a != nullptr) hipblasLtMatrixLayoutDestroy(pl.a);
  if (pl.b != nullptr) hipblasLtMatrixLayoutDestroy(pl.b);
  if (pl.d != nullptr) hipblasLtMatrixLayoutDestroy(pl.d);
  if (pl.desc != nullptr) hipblasLtMatmulDescDestroy(pl.desc);
  pl = GemmPlan{};
}

}  // namespace

bool gemm_x_wt_supported(int64_t M, int64_t N, int64_t K, int64_t ldx, int dtype, bool bias, bool alpha_vector) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return false;
  if (handle_for_device(dev) == nullptr) return false;
  const GemmShape key{dev, M, N, K, ldx, dtype, bias, alpha_vector};
  thread_local std::vector<std::pair<GemmShape, bool>> known;
  for (const auto& e : known)
    if (e.first == key) return e.second;
  GemmPlan pl{};
  // the bias pointer is an attribute the heuristic does not dereference
  const void* dummy_bias = bias ? reinterpret_cast<const void*>(static_cast<uintptr_t>(256)) : nullptr;
  hipblasLtMatmulAlgo_t algos[kCandidates];
  const bool ok = build_descriptors(key, pl, dummy_bias) && workspace_free_candidates(pl, algos) > 0;
  destroy_plan(pl);
  known.emplace_back(key, ok);
  return ok;
}

int gemm_x_wt(const uint16_t* x, int64_t ldx, const uint16_t* wt, const uint16_t* bias, uint16_t* y, int64_t M,
              int64_t N, int64_t K, int dtype, const float* alpha_vec, hipStream_t st, const GemmPrelude* prelude) {
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GRINQH_ERR_HIP;
  hipblasLtHandle_t h = handle_for_device(dev);
  if (h == nullptr) return GRINQH_ERR_HIP;
  thread_local std::vector<GemmPlan> plans;
  const GemmShape key{dev, M, N, K, ldx, dtype, bias != nullptr, alpha_vec != nullptr};
  GemmPlan* pl = nullptr;
  for (GemmPlan& q : plans)
    if (q.shape == key) pl = &q;
  const float alpha = 1.f, beta = 0.f;
  const float* pa = alpha_vec != nullptr ? alpha_vec : &alpha;
  const float* pb = &beta;
  if (pl == nullptr) {
    GemmPlan q{};
    if (!make_plan(key, q, GemmCall{wt, x, pa, pb, y, bias, st, prelude})) {
      destroy_plan(q);
      return GRINQH_ERR_HIP;
    }
    plans.push_back(q);
    pl = &plans.back();
  }
  if (bias != nullptr) {
    const void* bp = bias;
    if (hipblasLtMatmulDescSetAttribute(pl->desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bp, sizeof(bp)) !=
        HIPBLAS_STATUS_SUCCESS) {
      blas_failed("bias pointer", -1, key);
      return GRINQH_ERR_HIP;
    }
  }
  const hipblasStatus_t s = hipblasLtMatmul(h, pl->desc, pa, wt, pl->a, x, pl->b, pb, y, pl->d, y, pl->d,
                                            &pl->algo, nullptr, 0, st);
  if (s != HIPBLAS_STATUS_SUCCESS) {
    blas_failed("matmul", s, key);
    return GRINQH_ERR_HIP;
  }
  return GRINQH_OK;
}

}  // namespace grinqh
