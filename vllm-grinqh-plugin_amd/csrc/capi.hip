// extern "C" entry points of libgrinqh_hip.so (declared in include/grinqh.h):
// argument validation, workspace carving and kernel selection.
#include <stdlib.h>
#include <string.h>

#include <cstdlib>
#include <cstring>

#include <mutex>

#include "grinqh_common.h"
#include "grinqh_launch.h"

using namespace grinqh;

// Scratch of the allocation-free entry point (see scratch_on_current_device).
static __device__ __align__(256) unsigned char scratch[GRINQH_NOALLOC_SCRATCH_BYTES];

namespace {

constexpr int kAbiVersion = 1;
constexpr int64_t kDecodeMaxRows = 64;     // rows handled by one decode launch

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

inline bool valid_bits(int b) { return b == 2 || b == 4 || b == 6 || b == 8; }
inline bool valid_dtype(int d) { return d == GRINQH_DTYPE_F16 || d == GRINQH_DTYPE_BF16; }
inline bool aligned(const void* p, size_t a) { return (reinterpret_cast<uintptr_t>(p) % a) == 0; }
inline size_t round_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

// One-shot kernel timing events (grinqh_time_next_product).
struct KernelEvents {
  std::mutex mu;
  hipEvent_t before = nullptr, after = nullptr;
};
KernelEvents g_events;

}  // namespace

namespace grinqh {
thread_local KernelTiming t_kernel_timing;
}  // namespace grinqh

namespace {

// Hands an armed one-shot timer to this thread's next main-kernel launch.
void arm_kernel_timing() {
  std::lock_guard<std::mutex> lock(g_events.mu);
  if (g_events.before != nullptr) {
    t_kernel_timing = KernelTiming{g_events.before, g_events.after};
    g_events.before = g_events.after = nullptr;
  }
}

struct WorkspaceLayout {
  size_t counter_off, sigma_off, partial_off, total;
  // library-GEMM prefill (when either dtype may take it): graded statistic
  // partials and non-finite row flags, then the dense weight [N][K] -- after
  // the regions the fused prefill uses
  size_t chunk_off, flag_off, range_off, wt_off;
  bool library_gemm;
  bool tall;       // the large-batch prefill kernel serves the product (prefill_tall.hip)
  TallPlan tall_plan;
  size_t xt_off;   // its repacked activations (after the partial sums)
  DecodePlan plan;
};

// Which kernel serves a large batch that both can.  Measured on MI355X
// (random fp16 data, kernel times): the dense weight plus the library GEMM
// wins from 1024 rows on every Llama-3-8B shape and at 512 rows for the
// smaller weights (qkv, o_proj); the hand-written large-batch kernel wins at
// 512 rows for gate_up and down (132 vs 166 us, 104 vs 119 us), where the
// library path's dequantization pass is a large share.  GRINQH_PREFILL=tall
// or =library forces one (read on every call, so a test can pin a path).
bool prefill_prefers_library(int64_t M, int64_t K, int64_t N) {
  const char* e = std::getenv("GRINQH_PREFILL");
  if (e != nullptr && std::strcmp(e, "tall") == 0) return false;
  if (e != nullptr && std::strcmp(e, "library") == 0) return true;
  return M > 512 || K * N < ((int64_t)1 << 25);
}

// Plan of one launch of mc rows: the GEMV kernel up to kGemvMaxRows rows, the
// decode kernel above.  group_size 32 gives the largest GEMV workspace.
DecodePlan plan_launch(int64_t mc, int64_t K, int64_t N, int64_t group_size) {
  return mc <= kGemvMaxRows ? plan_gemv(mc, K, N, group_size) : plan_decode(mc, K, N);
}
int launch_main(const DecodeParams& p, const DecodePlan& plan, int max_bits, int dtype, bool dense,
                hipStream_t st) {
  return p.M <= kGemvMaxRows ? launch_gemv(p, plan, max_bits, dtype, dense, st)
                             : launch_decode(p, plan, max_bits, dtype, dense, st);
}

// [split-K counters (kCounterBytes, zero between calls) | sigma (K floats,
// graded batches above kDecodeMaxRows) | split-K partials | repacked x of
// the large-batch kernel, or the library-GEMM regions].  The counters sit at
// offset 0 for every shape, so a workspace shared by calls of different
// shapes keeps them zero.  The size does not depend on the dtype: when either
// dtype may take the library path (bf16 from fewer rows) its regions follow
// those of the fused kernel, so either path runs from the same workspace.
//
// A prefill takes the library path where prefill_prefers_library says so and
// the library has an algorithm for the shape, else the large-batch kernel
// where it applies, else the fused kernel; without a workspace
// (allow_library = false) the large-batch kernel whenever it applies.  The
// large-batch kernel's shape conditions on K and N are known to the workspace
// query; the group size and ldx are not, so the partial-sum region covers
// both the large-batch kernel's split (within `budget`, the allocation-free
// entry point's scratch; 0: a caller-sized workspace) and the fused kernel's,
// so that any call of the queried (M, K, N, mode) runs in it.
WorkspaceLayout layout_for(int64_t M, int64_t K, int64_t N, int mode, bool allow_library = true,
                           int64_t ldx = -1, int gs = -1, size_t budget = 0) {
  WorkspaceLayout w{};
  size_t partial = 0, xt = 0;
  const bool g = mode == GRINQH_MODE_UNION;
  const bool need_sigma = g && M > kDecodeMaxRows;  // the prefill's statistic pass
  const size_t head = kCounterBytes + (need_sigma ? round_up((size_t)K * sizeof(float), 256) : 0);
  // where the large-batch kernel applies the library path needs an algorithm
  // for both dtypes (the layout serves either); elsewhere for either
  const bool lib_f16 = use_library_gemm(M, K, N, GRINQH_DTYPE_F16), lib_bf16 = use_library_gemm(M, K, N, GRINQH_DTYPE_BF16);
  const bool tall_fits = M > kDecodeMaxRows && prefill_tall_applies(M, K, N, K, 128);
  const bool lib_first = allow_library && M > kDecodeMaxRows &&
                         (tall_fits ? lib_f16 && lib_bf16 && prefill_prefers_library(M, K, N) : lib_f16 || lib_bf16);
  bool tall_shape = false;
  if (M <= kDecodeMaxRows) {
    w.plan = plan_launch(M > 0 ? M : 1, K, N, 32);
    partial = w.plan.splits > 1 ? w.plan.workspace : 0;
  } else {  // prefill: partial sums only when its grid is split over K
    tall_shape = !lib_first && tall_fits;
    xt = tall_shape ? round_up(tall_x_bytes(M, K), 256) : 0;
    if (tall_shape && budget != 0 && head + xt > budget) tall_shape = false, xt = 0;  // no room for x repacked
    w.tall = tall_shape && ldx >= 0 && gs > 0 && prefill_tall_applies(M, K, N, ldx, gs);
    if (tall_shape) {
      const size_t room = budget == 0 ? kMaxPrefillPartialBytes : budget - head - xt;
      w.tall_plan = plan_tall(M, K, N, room);
      partial = tall_partial_bytes(w.tall_plan, M, N);
    }
    if (!w.tall) {  // the fused kernel (a call that cannot take the large-batch kernel)
      const int splits = prefill_splits(M, K, N);
      const size_t fused = splits > 1 ? (size_t)splits * (size_t)M * (size_t)N * sizeof(float) : 0;
      partial = fused > partial ? fused : partial;
    }
  }
  w.counter_off = 0;
  w.sigma_off = kCounterBytes;
  w.partial_off = head;
  w.xt_off = round_up(w.partial_off + partial, 256);
  w.total = (partial == 0 && !need_sigma && xt == 0) ? 0 : w.xt_off + xt;
  w.library_gemm = allow_library && !tall_shape && M > kDecodeMaxRows &&
                   (use_library_gemm(M, K, N, GRINQH_DTYPE_F16) || use_library_gemm(M, K, N, GRINQH_DTYPE_BF16));
  if (w.library_gemm) {  // (no repacked x: the large-batch kernel cannot take these shapes)
    const int64_t chunks = (M + sigma_chunk_rows(M) - 1) / sigma_chunk_rows(M);
    w.chunk_off = round_up(w.partial_off + partial, 256);
    w.flag_off = w.chunk_off + (g ? round_up((size_t)chunks * (size_t)K * sizeof(float), 256) : 0);
    // graded: the overflow guard's scale-range slots, then the GEMM's alpha vector
    w.range_off = w.flag_off + (g ? round_up((size_t)((K + 255) / 256) * (size_t)M, 256) : 0);
    w.wt_off = w.range_off + (g ? round_up((size_t)scale_range_slots(K) * 4, 256) + round_up((size_t)N * 4, 256) : 0);
    w.total = w.wt_off + round_up((size_t)N * (size_t)K * 2, 256);
  }
  return w;
}

int check_product_args(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                       const void* planes, const void* scale, void* y, int max_bits, int group_size) {
  if (!valid_dtype(dtype) || !valid_bits(max_bits)) return GRINQH_ERR_INVALID;
  if (M < 0 || K <= 0 || N <= 0 || K % 32 != 0 || N % 16 != 0) return GRINQH_ERR_INVALID;
  if (group_size <= 0 || group_size % 32 != 0) return GRINQH_ERR_INVALID;
  if (K > (int64_t)1 << 30 || N > (int64_t)1 << 24 || M > (int64_t)1 << 30) return GRINQH_ERR_INVALID;
  if (M > 0 && (x == nullptr || planes == nullptr || scale == nullptr || y == nullptr)) return GRINQH_ERR_INVALID;
  if (ldx < K || ldx % 8 != 0 || !aligned(x, 16) || !aligned(planes, 4)) return GRINQH_ERR_INVALID;
  if (!aligned(y, 8) || !aligned(scale, 2)) return GRINQH_ERR_INVALID;
  // plane words are addressed with 32-bit byte offsets (bit 31 reserved)
  if (K * (max_bits / 2) * (N / 16) * 4 >= ((int64_t)1 << 31)) return GRINQH_ERR_INVALID;
  // the GEMV / decode kernels address the x rows of one launch (at most
  // kDecodeMaxRows) through 32-bit buffer offsets as well
  const int64_t rows_per_launch = M < kDecodeMaxRows ? M : kDecodeMaxRows;
  if (rows_per_launch * ldx * 2 >= ((int64_t)1 << 31)) return GRINQH_ERR_INVALID;
  return GRINQH_OK;
}

// The fused prefill kernel addresses all of x through one 32-bit buffer
// descriptor; only the library-GEMM path (64-bit addressing throughout) takes
// larger activations.
bool x_fits_fused_prefill(int64_t M, int64_t ldx) { return M * ldx * 2 < ((int64_t)1 << 31); }

// M > kDecodeMaxRows: the large-batch kernel where the layout chose it
// (wl.tall), else the library-GEMM path (use_library_gemm, when the library
// has an algorithm without workspace for the shape), else one prefill launch
// over the whole batch, the wide-tile kernel where it applies
// (prefill_wide_applies) or the fused prefill kernel (graded batches first
// reduce the union statistic over all M rows).  The workspace layout holds
// the fused kernel's regions in front of the library path's, so either runs.
int run_prefill(const DecodeParams& d, const uint16_t* xs, uint16_t* ys, int64_t M, int dtype, int max_bits,
                bool graded, char* ws, const WorkspaceLayout& wl, hipStream_t st) {
  if (wl.tall) {  // the large-batch kernel: x repacked (graded: the batch statistic first)
    uint16_t* xt = reinterpret_cast<uint16_t*>(ws + wl.xt_off);
    int rc = launch_repack_x(xs, d.ldx, (int)M, d.K, xt, st);
    if (rc != GRINQH_OK) return rc;
    PrefillParams p{};
    p.x = xt;
    p.ldx = d.K;
    p.planes = d.planes;
    p.scale = d.scale;
    p.bias = d.bias;
    p.y = ys;
    p.thr = d.thr;
    p.M = (int)M;
    p.K = d.K;
    p.N = d.N;
    p.NW = d.NW;
    p.gs = d.gs;
    p.splits = wl.tall_plan.splits;
    p.dp_tiles = wl.tall_plan.dp_tiles;
    p.partial = p.splits > 1 ? reinterpret_cast<float*>(ws + wl.partial_off) : nullptr;
    p.counters = p.splits > 1 ? reinterpret_cast<uint32_t*>(ws + wl.counter_off) : nullptr;
    if (graded) {  // each K row's grade word, in the statistic's region (K words)
      uint32_t* grades = reinterpret_cast<uint32_t*>(ws + wl.sigma_off);
      rc = launch_grade_words(xs, d.ldx, (int)M, d.K, dtype, max_bits, d.thr, grades, st);
      if (rc != GRINQH_OK) return rc;
      p.grades = grades;
    }
    arm_kernel_timing();
    rc = launch_prefill_tall(p, wl.tall_plan, max_bits, dtype, !graded, st);
    t_kernel_timing = KernelTiming{};
    return rc;
  }
  if (wl.library_gemm && use_library_gemm(M, d.K, d.N, dtype) &&
      gemm_x_wt_supported(M, d.N, d.K, d.ldx, dtype, /*bias=*/false, graded && dtype == GRINQH_DTYPE_F16) &&
      (d.bias == nullptr || aligned(d.bias, 16))) {  // the (graded) weight once, then the library GEMM
    // an error a library left in this thread's last-error slot must not be
    // taken for a failure of the launches below
    (void)hipGetLastError();
    uint16_t* wt = reinterpret_cast<uint16_t*>(ws + wl.wt_off);
    float* sigma = graded ? reinterpret_cast<float*>(ws + wl.sigma_off) : nullptr;
    uint8_t* flags = reinterpret_cast<uint8_t*>(ws + wl.flag_off);
    // graded fp16: the overflow guard of the dense weight (scale-range slots, alpha on the device)
    const bool guard = graded && dtype == GRINQH_DTYPE_F16;
    uint32_t* slots = guard ? reinterpret_cast<uint32_t*>(ws + wl.range_off) : nullptr;
    float* alpha =
        guard ? reinterpret_cast<float*>(ws + wl.range_off + round_up((size_t)scale_range_slots(d.K) * 4, 256))
              : nullptr;
    const int64_t n_scale = (int64_t)((d.K + d.gs - 1) / d.gs) * d.N;
    int rc = graded ? launch_sigma_chunks(xs, d.ldx, (int)M, d.K, dtype, reinterpret_cast<float*>(ws + wl.chunk_off),
                                          flags, sigma, guard ? d.scale : nullptr, n_scale, slots, st)
                    : GRINQH_OK;
    if (rc != GRINQH_OK) return rc;
    auto dequant = [&](hipStream_t s) {
      return launch_dequant_nk(d.planes, d.scale, wt, d.K, d.N, d.gs, max_bits, dtype, sigma, d.thr, slots, alpha, s);
    };
    arm_kernel_timing();
    rc = dequant(st);
    t_kernel_timing = KernelTiming{};
    const GemmPrelude prelude = dequant;
    // the GEMM rounds its output once; the bias follows as its own rounding
    // (cast, then add, as the reference's y.add_(bias) after the matmul)
    if (rc == GRINQH_OK) rc = gemm_x_wt(xs, d.ldx, wt, nullptr, ys, M, d.N, d.K, dtype, alpha, st, &prelude);
    if (rc == GRINQH_OK && d.bias != nullptr) {
      (void)hipGetLastError();  // a library call may leave an error in this thread's slot
      rc = launch_add_bias_rows(ys, d.bias, M, d.N, dtype, st);
    }
    if (rc == GRINQH_OK && graded) {
      (void)hipGetLastError();  // the GEMM's library calls may leave one behind as well
      rc = launch_nonfinite_rows_to_nan(flags, (int)M, d.K, ys, d.N, dtype, st);
    }
    return rc;
  }
  if (!x_fits_fused_prefill(M, d.ldx)) return GRINQH_ERR_INVALID;  // x of 2 GiB or more: split the batch
  // neither the large-batch kernel nor the library path: the wide-tile
  // kernel where its grid fills the GPU, else the fused prefill kernel
  const bool wide = prefill_wide_applies(M, d.K, d.N, d.ldx, d.gs, dtype);
  PrefillParams p{};
  p.x = xs;
  p.ldx = d.ldx;
  p.planes = d.planes;
  p.scale = d.scale;
  p.bias = d.bias;
  p.y = ys;
  p.thr = d.thr;
  p.M = (int)M;
  p.K = d.K;
  p.N = d.N;
  p.NW = d.NW;
  p.gs = d.gs;
  p.sigma = nullptr;
  p.splits = wide ? 1 : prefill_splits(M, d.K, d.N);
  p.partial = p.splits > 1 ? reinterpret_cast<float*>(ws + wl.partial_off) : nullptr;
  if (graded) {  // the batch statistic the rows are graded on
    float* sigma = reinterpret_cast<float*>(ws + wl.sigma_off);
    const int rc = launch_sigma(xs, d.ldx, (int)M, d.K, dtype, sigma, st);
    if (rc != GRINQH_OK) return rc;
    p.sigma = sigma;
  }
  arm_kernel_timing();
  int splits_run = 1;
  int rc = wide ? launch_prefill_wide(p, max_bits, !graded, st)
                : launch_prefill(p, max_bits, dtype, !graded, st, &splits_run);
  t_kernel_timing = KernelTiming{};
  if (rc != GRINQH_OK) return rc;
  if (splits_run > 1) {  // add the K ranges in order, cast, bias
    DecodeParams r = d;
    r.M = (int)M;
    r.y = ys;
    r.partial = p.partial;
    rc = launch_splitk_reduce(r, splits_run, dtype, st);
  }
  return rc;
}

// allow_library = false keeps every batch on the fused kernels (no dense
// weight buffer), and a workspace too small for the product's layout is
// reported as GRINQH_ERR_SCRATCH instead of GRINQH_ERR_WORKSPACE (the
// allocation-free entry point's fixed scratch).
int run_product(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype, const void* planes,
                const void* scale, const void* bias, void* y, int max_bits, int group_size,
                const float* thresholds, int mode, void* workspace, size_t ws_bytes, void* stream,
                bool allow_library = true, const float* sigma_given = nullptr) {
  int rc = check_product_args(x, M, K, ldx, N, dtype, planes, scale, y, max_bits, group_size);
  if (rc != GRINQH_OK) return rc;
  if (mode != GRINQH_MODE_REFERENCE && mode != GRINQH_MODE_UNION && mode != GRINQH_MODE_DENSE)
    return GRINQH_ERR_INVALID;
  if (M == 0) return GRINQH_OK;
  const bool graded = mode == GRINQH_MODE_UNION || (mode == GRINQH_MODE_REFERENCE && M == 1);
  if (graded && thresholds == nullptr) return GRINQH_ERR_INVALID;

  const int mode_l = graded ? GRINQH_MODE_UNION : GRINQH_MODE_DENSE;
  WorkspaceLayout wl = layout_for(M, K, N, mode_l, allow_library, ldx, group_size, allow_library ? 0 : ws_bytes);
  // The allocation-free entry point's fixed scratch may not hold a decode
  // launch's split-K partial sums (a large K forces many K ranges, and the
  // partial sums grow with the rows): then the rows run in chunks (halving
  // until one chunk's layout fits), graded on the statistic of the whole
  // batch, reduced once into the scratch past the chunks' layout.  With one
  // row every valid shape fits.
  int64_t rows_per_launch = kDecodeMaxRows;
  size_t sigma_off = 0;
  if (!allow_library && M <= kDecodeMaxRows && wl.total > ws_bytes) {
    const size_t sig_bytes = graded && sigma_given == nullptr ? round_up((size_t)K * sizeof(float), 256) : 0;
    auto need = [&](const WorkspaceLayout& w) {
      return round_up(w.total > kCounterBytes ? w.total : kCounterBytes, 256) + sig_bytes;
    };
    int64_t mc = M;
    while (mc > 1 && need(wl) > ws_bytes) {
      mc = (mc + 1) / 2;
      wl = layout_for(mc, K, N, mode_l, false, ldx, group_size, ws_bytes);
    }
    if (need(wl) > ws_bytes) return GRINQH_ERR_SCRATCH;
    rows_per_launch = mc;
    sigma_off = need(wl) - sig_bytes;
  }
  if (wl.total > 0 && (workspace == nullptr || ws_bytes < wl.total || !aligned(workspace, 256)))
    return allow_library ? GRINQH_ERR_WORKSPACE : GRINQH_ERR_SCRATCH;
  hipStream_t st = as_stream(stream);
  char* ws = static_cast<char*>(workspace);

  DecodeParams p{};
  p.planes = static_cast<const uint32_t*>(planes);
  p.scale = static_cast<const uint16_t*>(scale);
  p.bias = static_cast<const uint16_t*>(bias);
  p.ldx = ldx;
  p.K = (int)K;
  p.N = (int)N;
  p.NW = (int)(N / 16);
  p.gs = group_size;
  for (int i = 0; i < 4; ++i) p.thr.t[i] = graded ? thresholds[i] : 0.f;
  p.partial = ws ? reinterpret_cast<float*>(ws + wl.partial_off) : nullptr;
  p.sigma = nullptr;

  const uint16_t* xs = static_cast<const uint16_t*>(x);
  uint16_t* ys = static_cast<uint16_t*>(y);
  if (M > kDecodeMaxRows) return run_prefill(p, xs, ys, M, dtype, max_bits, graded, ws, wl, st);
  if (graded && sigma_given != nullptr) {  // the producer's chunk maxima (grinqh_*_sigma)
    p.sigma = sigma_given;
    p.sigma_chunks = (int)((M + kSigmaChunkRows - 1) / kSigmaChunkRows);
  } else if (graded && rows_per_launch < M) {  // row chunks: grade on the whole batch's statistic
    float* sig = reinterpret_cast<float*>(ws + sigma_off);
    rc = launch_sigma(xs, ldx, (int)M, (int)K, dtype, sig, st);
    if (rc != GRINQH_OK) return rc;
    p.sigma = sig;
    p.sigma_chunks = 1;
  }  // else the GEMV and decode kernels reduce the batch statistic of their rows themselves
  for (int64_t m0 = 0; m0 < M; m0 += rows_per_launch) {
    const int64_t mc = (M - m0) < rows_per_launch ? (M - m0) : rows_per_launch;
    const DecodePlan plan = plan_launch(mc, K, N, group_size);
    p.x = xs + m0 * ldx;
    p.y = ys + m0 * N;
    p.M = (int)mc;
    p.splits = plan.splits;
    p.tiles_per_split = plan.tiles_per_split;
    const int64_t block_cols = mc <= kGemvMaxRows ? 1024 : 256;  // logical columns per column block
    p.counters =
        splitk_in_kernel(plan, mc, N, block_cols) ? reinterpret_cast<uint32_t*>(ws + wl.counter_off) : nullptr;
    if (m0 == 0) arm_kernel_timing();
    rc = launch_main(p, plan, max_bits, dtype, !graded, st);
    t_kernel_timing = KernelTiming{};
    if (rc != GRINQH_OK) return rc;
    if (plan.splits > 1 && p.counters == nullptr) {
      rc = launch_splitk_reduce(p, plan.splits, dtype, st);
      if (rc != GRINQH_OK) return rc;
    }
  }
  return GRINQH_OK;
}

// ---- allocation-free entry point (grinqh_gemm_or_gemv_noalloc)
//
// Its split-K counters, partial sums and grading statistic live in this
// file-scope device array; every GPU the library runs on holds its own copy
// until the process ends.  In host code `scratch` names a host-side stand-in,
// never device memory: its device address is looked up once per device with
// hipGetSymbolAddress (that device current) and only that address is used.
constexpr size_t kScratchBytes = GRINQH_NOALLOC_SCRATCH_BYTES;

constexpr int kMaxDevices = 64;
struct ScratchSlot {
  void* ptr = nullptr;   // device address of `scratch` on this device
  bool cleared = false;  // counter area cleared on a stream once
};
std::mutex g_scratch_mu;
ScratchSlot g_scratch[kMaxDevices];

__global__ void clear_words_kernel(uint32_t* p, int n) {
  const int i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) p[i] = 0u;
}

// The scratch address on the current device.  The first call on a device
// also clears the split-K counter area with a fill kernel on `st` (device
// globals start zeroed; this makes it so whatever the loader did), which a
// graph under capture may record: it only ever writes zeros where every
// call leaves zeros.
int scratch_on_current_device(void** out, hipStream_t st) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return GRINQH_ERR_HIP;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  ScratchSlot& slot = g_scratch[dev];
  if (slot.ptr == nullptr) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) return GRINQH_ERR_HIP;
    slot.ptr = p;
  }
  if (!slot.cleared) {
    constexpr int words = (int)(kCounterBytes / 4);
    hipLaunchKernelGGL(clear_words_kernel, dim3((words + 255) / 256), dim3(256), 0, st,
                       static_cast<uint32_t*>(slot.ptr), words);
    if (hipGetLastError() != hipSuccess) return GRINQH_ERR_HIP;
    slot.cleared = true;
  }
  *out = slot.ptr;
  return GRINQH_OK;
}

}  // namespace

extern "C" {

int grinqh_abi_version(void) { return kAbiVersion; }

const char* grinqh_status_string(int status) {
  switch (status) {
    case GRINQH_OK: return "ok";
    case GRINQH_ERR_INVALID: return "invalid argument (shape, dtype, bit width, alignment or mode)";
    case GRINQH_ERR_HIP: return "HIP kernel launch failed";
    case GRINQH_ERR_WORKSPACE: return "workspace missing, misaligned or too small";
    case GRINQH_ERR_SCRATCH:
      return "problem needs more scratch than the allocation-free entry point holds (GRINQH_NOALLOC_SCRATCH_BYTES)";
    default: return "unknown status";
  }
}

int grinqh_pack_planes(const void* codes_u8, void* planes_u32, int64_t K, int64_t N, int max_bits,
                       void* stream) {
  if (!valid_bits(max_bits) || K < 0 || N < 0 || N % 16 != 0) return GRINQH_ERR_INVALID;
  if (K * N == 0) return GRINQH_OK;
  if (codes_u8 == nullptr || planes_u32 == nullptr || !aligned(codes_u8, 16) || !aligned(planes_u32, 4))
    return GRINQH_ERR_INVALID;
  if (K > INT32_MAX || N > INT32_MAX) return GRINQH_ERR_INVALID;
  return launch_pack_planes(static_cast<const uint32_t*>(codes_u8), static_cast<uint32_t*>(planes_u32), (int)K,
                            (int)N, max_bits, as_stream(stream));
}

int grinqh_prepare_weight(const void* w_int8, void* planes_u32, int64_t K, int64_t N, int max_bits,
                          void* stream) {
  if (!valid_bits(max_bits) || K < 0 || N < 0 || N % 16 != 0) return GRINQH_ERR_INVALID;
  if (K * N == 0) return GRINQH_OK;
  if (w_int8 == nullptr || planes_u32 == nullptr || !aligned(planes_u32, 4)) return GRINQH_ERR_INVALID;
  if (K > INT32_MAX || N > INT32_MAX) return GRINQH_ERR_INVALID;
  return launch_prepare_weight(static_cast<const int8_t*>(w_int8), static_cast<uint32_t*>(planes_u32), (int)K,
                               (int)N, max_bits, as_stream(stream));
}

int grinqh_unpack_planes(const void* planes_u32, const int64_t* rows, int64_t n_rows, void* codes_u32, int64_t K,
                         int64_t N, int bit_level, void* stream) {
  if (bit_level < 1 || bit_level > 4 || n_rows < 0 || K < 0 || N < 0 || N % 16 != 0) return GRINQH_ERR_INVALID;
  if (n_rows * N == 0) return GRINQH_OK;
  if (planes_u32 == nullptr || rows == nullptr || codes_u32 == nullptr || !aligned(codes_u32, 16))
    return GRINQH_ERR_INVALID;
  if (n_rows > INT32_MAX || N > INT32_MAX) return GRINQH_ERR_INVALID;
  return launch_unpack_planes(static_cast<const uint32_t*>(planes_u32), rows, static_cast<uint32_t*>(codes_u32),
                              (int)n_rows, (int)N, bit_level, as_stream(stream));
}

int grinqh_dequantize(const void* planes_u32, const void* scale, void* out, int64_t K, int64_t N, int max_bits,
                      int group_size, int dtype, void* stream) {
  if (!valid_bits(max_bits) || !valid_dtype(dtype) || K < 0 || N < 0 || N % 16 != 0) return GRINQH_ERR_INVALID;
  if (scale != nullptr && group_size <= 0) return GRINQH_ERR_INVALID;
  if (K * N == 0) return GRINQH_OK;
  if (planes_u32 == nullptr || out == nullptr) return GRINQH_ERR_INVALID;
  if (K > INT32_MAX || N > INT32_MAX) return GRINQH_ERR_INVALID;
  return launch_dequant(static_cast<const uint32_t*>(planes_u32), static_cast<const uint16_t*>(scale), out, (int)K,
                        (int)N, max_bits, group_size > 0 ? group_size : 1, dtype, as_stream(stream));
}

int grinqh_grade(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype, int max_bits,
                 const float thresholds[4], uint8_t* zone_bits, int32_t* beta, void* stream) {
  if (!valid_bits(max_bits) || !valid_dtype(dtype) || M < 1 || K < 0 || ldx < K) return GRINQH_ERR_INVALID;
  if (K == 0) return GRINQH_OK;
  if (x == nullptr || thresholds == nullptr || zone_bits == nullptr) return GRINQH_ERR_INVALID;
  if (K > INT32_MAX || M > INT32_MAX) return GRINQH_ERR_INVALID;
  return launch_grade(static_cast<const uint16_t*>(x), ldx, (int)M, (int)K, thresholds, max_bits, dtype, zone_bits,
                      beta, as_stream(stream));
}

size_t grinqh_workspace_bytes(int64_t M, int64_t K, int64_t N, int max_bits, int mode) {
  (void)max_bits;
  if (M <= 0 || K <= 0 || N <= 0) return 0;
  const bool graded = mode == GRINQH_MODE_UNION || (mode == GRINQH_MODE_REFERENCE && M == 1);
  return layout_for(M, K, N, graded ? GRINQH_MODE_UNION : GRINQH_MODE_DENSE).total;
}

int grinqh_gemm_or_gemv(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                        const void* planes_u32, const void* scale, const void* bias, void* y, int max_bits,
                        int group_size, const float thresholds[4], int mode, void* workspace,
                        size_t workspace_bytes, void* stream) {
  return run_product(x, M, K, ldx, N, dtype, planes_u32, scale, bias, y, max_bits, group_size, thresholds, mode,
                     workspace, workspace_bytes, stream);
}

int grinqh_gemv_batch_union(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                            const void* planes_u32, const void* scale, const void* bias, void* y, int max_bits,
                            int group_size, const float thresholds[4], void* workspace, size_t workspace_bytes,
                            void* stream) {
  return run_product(x, M, K, ldx, N, dtype, planes_u32, scale, bias, y, max_bits, group_size, thresholds,
                     GRINQH_MODE_UNION, workspace, workspace_bytes, stream);
}

int grinqh_prefill_dense(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                         const void* planes_u32, const void* scale, const void* bias, void* y, int max_bits,
                         int group_size, void* workspace, size_t workspace_bytes, void* stream) {
  return run_product(x, M, K, ldx, N, dtype, planes_u32, scale, bias, y, max_bits, group_size, nullptr,
                     GRINQH_MODE_DENSE, workspace, workspace_bytes, stream);
}

int grinqh_gemm_or_gemv_noalloc(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                                const void* planes_u32, const void* scale, const void* bias, void* y, int max_bits,
                                int group_size, const float thresholds[4], int mode, void* stream) {
  // arguments first (shapes, mode, thresholds): an invalid call touches no device state
  int rc = check_product_args(x, M, K, ldx, N, dtype, planes_u32, scale, y, max_bits, group_size);
  if (rc != GRINQH_OK) return rc;
  if (mode != GRINQH_MODE_REFERENCE && mode != GRINQH_MODE_UNION && mode != GRINQH_MODE_DENSE)
    return GRINQH_ERR_INVALID;
  if (M == 0) return GRINQH_OK;
  const bool graded = mode == GRINQH_MODE_UNION || (mode == GRINQH_MODE_REFERENCE && M == 1);
  if (graded && thresholds == nullptr) return GRINQH_ERR_INVALID;
  void* ws = nullptr;
  rc = scratch_on_current_device(&ws, as_stream(stream));
  if (rc != GRINQH_OK) return rc;
  return run_product(x, M, K, ldx, N, dtype, planes_u32, scale, bias, y, max_bits, group_size, thresholds, mode, ws,
                     kScratchBytes, stream, /*allow_library=*/false);
}

int grinqh_rmsnorm_sigma(const void* x, int64_t M, int64_t K, int64_t ldx, const void* residual, void* residual_out,
                         const void* weight, float eps, void* y, float* sigma_chunks, int dtype, void* stream) {
  if (!valid_dtype(dtype) || M < 0 || K <= 0 || K % 8 != 0 || ldx < K || ldx % 8 != 0) return GRINQH_ERR_INVALID;
  if (K > ((int64_t)1 << 30) || M > ((int64_t)1 << 30) || !(eps >= 0.f)) return GRINQH_ERR_INVALID;
  if (M == 0) return GRINQH_OK;
  if (x == nullptr || weight == nullptr || y == nullptr || sigma_chunks == nullptr) return GRINQH_ERR_INVALID;
  if ((residual == nullptr) != (residual_out == nullptr)) return GRINQH_ERR_INVALID;
  if (!aligned(x, 16) || !aligned(weight, 16) || !aligned(y, 16) || !aligned(sigma_chunks, 4)) return GRINQH_ERR_INVALID;
  if (residual != nullptr && (!aligned(residual, 16) || !aligned(residual_out, 16) || residual_out == residual))
    return GRINQH_ERR_INVALID;
  if (y == x || y == residual) return GRINQH_ERR_INVALID;  // every block reads whole rows of both
  return launch_rmsnorm_sigma(static_cast<const uint16_t*>(x), ldx, static_cast<const uint16_t*>(residual),
                              static_cast<uint16_t*>(residual_out), static_cast<const uint16_t*>(weight), eps,
                              static_cast<uint16_t*>(y), sigma_chunks, (int)M, (int)K, dtype, as_stream(stream));
}

int grinqh_silu_mul_sigma(const void* gate_up, int64_t M, int64_t F, int64_t ld, void* y, float* sigma_chunks,
                          int dtype, void* stream) {
  if (!valid_dtype(dtype) || M < 0 || F <= 0 || F % 8 != 0 || ld < 2 * F || ld % 8 != 0) return GRINQH_ERR_INVALID;
  if (F > ((int64_t)1 << 30) || M > ((int64_t)1 << 30)) return GRINQH_ERR_INVALID;
  if (M == 0) return GRINQH_OK;
  if (gate_up == nullptr || y == nullptr || sigma_chunks == nullptr) return GRINQH_ERR_INVALID;
  if (!aligned(gate_up, 16) || !aligned(y, 16) || !aligned(sigma_chunks, 4) || y == gate_up) return GRINQH_ERR_INVALID;
  return launch_silu_mul_sigma(static_cast<const uint16_t*>(gate_up), ld, static_cast<uint16_t*>(y), sigma_chunks,
                               (int)M, (int)F, dtype, as_stream(stream));
}

int grinqh_gemv_batch_union_sigma(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                                  const void* planes_u32, const void* scale, const void* bias, void* y, int max_bits,
                                  int group_size, const float thresholds[4], const float* sigma_chunks,
                                  void* workspace, size_t workspace_bytes, void* stream) {
  if (sigma_chunks == nullptr || !aligned(sigma_chunks, 4)) return GRINQH_ERR_INVALID;
  return run_product(x, M, K, ldx, N, dtype, planes_u32, scale, bias, y, max_bits, group_size, thresholds,
                     GRINQH_MODE_UNION, workspace, workspace_bytes, stream, /*allow_library=*/true, sigma_chunks);
}

int grinqh_product_kernel(int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype, int max_bits, int group_size,
                          int mode, int noalloc, int* rows_per_block, int* splits) {
  const void* nz = reinterpret_cast<const void*>(static_cast<uintptr_t>(256));  // stands for valid pointers
  if (M < 1 || check_product_args(nz, M, K, ldx, N, dtype, nz, nz, const_cast<void*>(nz), max_bits, group_size) !=
                   GRINQH_OK)
    return -GRINQH_ERR_INVALID;
  if (mode != GRINQH_MODE_REFERENCE && mode != GRINQH_MODE_UNION && mode != GRINQH_MODE_DENSE)
    return -GRINQH_ERR_INVALID;
  if (rows_per_block != nullptr) *rows_per_block = 0;
  if (splits != nullptr) *splits = 0;
  if (M <= kDecodeMaxRows) return M <= kGemvMaxRows ? GRINQH_KERNEL_GEMV : GRINQH_KERNEL_DECODE;
  const bool graded = mode == GRINQH_MODE_UNION;
  const bool allow_library = noalloc == 0;
  const WorkspaceLayout wl = layout_for(M, K, N, graded ? GRINQH_MODE_UNION : GRINQH_MODE_DENSE, allow_library, ldx,
                                        group_size, allow_library ? 0 : kScratchBytes);
  if (wl.tall) {
    if (rows_per_block != nullptr) *rows_per_block = 64 * wl.tall_plan.rt;
    if (splits != nullptr) *splits = wl.tall_plan.splits;
    return GRINQH_KERNEL_TALL;
  }
  // (the library's own algorithm query, made at run time on the device, can
  // still send such a call to the fused kernel)
  if (wl.library_gemm && use_library_gemm(M, K, N, dtype)) return GRINQH_KERNEL_LIBRARY;
  return GRINQH_KERNEL_FUSED;
}

int grinqh_time_next_product(void* event_before, void* event_after) {
  if ((event_before == nullptr) != (event_after == nullptr)) return GRINQH_ERR_INVALID;
  std::lock_guard<std::mutex> lock(g_events.mu);
  g_events.before = static_cast<hipEvent_t>(event_before);
  g_events.after = static_cast<hipEvent_t>(event_after);
  return GRINQH_OK;
}

}  // extern "C"
