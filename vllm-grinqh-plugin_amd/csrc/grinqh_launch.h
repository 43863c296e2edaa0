// Internal launch interface between the C ABI (capi.hip) and the kernel files.
#pragma once
#include <hip/hip_ext.h>
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

#include <functional>

#include "grinqh.h"

namespace grinqh {

struct GradeThresholds {
  float t[4];
};

// Upper bound on the split-K partial-sum area.
constexpr size_t kMaxPartialBytes = size_t(64) << 20;

struct DecodeParams {
  const uint16_t* x;
  int64_t ldx;
  const uint32_t* planes;
  const uint16_t* scale;
  const uint16_t* bias;
  uint16_t* y;
  GradeThresholds thr;
  int M, K, N, NW, gs;
  int splits;           // grid.y: K ranges
  int tiles_per_split;  // 32-row tiles per K range
  float* partial;       // [splits][M][N] fp32 when splits > 1
  const float* sigma;   // optional precomputed union statistic (else computed from x):
                        // sigma_chunks arrays of K column maxima whose maximum is sigma_k
  int sigma_chunks;     // arrays at sigma (1 for a plain [K] statistic)
  uint32_t* counters;   // per column block, zero on entry: the kernel completes split-K
                        // itself; nullptr: partial sums only, the reduce kernel follows
};

struct DecodePlan {
  int mt;      // 16-row m-tiles: 1, 2 or 4 (M <= 16, 32, 64)
  int splits;
  int tiles_per_split;
  int col_blocks;
  size_t workspace;  // partial-sum bytes, 0 if splits == 1
};

DecodePlan plan_decode(int64_t M, int64_t K, int64_t N);

// Split-K completion counters (one per column block) at the start of the
// workspace; larger column counts fall back to the reduce kernel.
constexpr int64_t kMaxCounters = 4096;
constexpr size_t kCounterBytes = size_t(kMaxCounters) * 4;
// Partial-sum bytes one column block's last K range may add up itself; above
// this one block's reads would outlast a separate, grid-wide reduction.
constexpr int64_t kInKernelReduceBytes = 64 << 10;
// Whether the main kernel completes split-K itself (DecodeParams::counters):
// whole 4-column chunks per column block, 32-bit partial-sum offsets and a
// small enough reduction.  cols = logical columns per column block.
inline bool splitk_in_kernel(const DecodePlan& pl, int64_t M, int64_t N, int64_t cols) {
  return pl.splits > 1 && (N / 16) % 4 == 0 && pl.col_blocks <= kMaxCounters &&
         (int64_t)pl.splits * M * N * 4 < ((int64_t)1 << 31) &&
         (int64_t)pl.splits * M * cols * 4 <= kInKernelReduceBytes;
}

// Main kernels: when plan.splits > 1 and p.counters is null the caller
// follows with launch_splitk_reduce.
int launch_decode(const DecodeParams& p, const DecodePlan& plan, int max_bits, int dtype, bool dense,
                  hipStream_t st);
// y = cast(sum over `splits` of partial[s][M][N]) (+ bias), ranges added in order
int launch_splitk_reduce(const DecodeParams& p, int splits, int dtype, hipStream_t st);

constexpr int64_t kTargetBlocks = 256;  // MI355X compute units

// GEMV path (M <= kGemvMaxRows): one word column per lane, 8-row tiles.
constexpr int64_t kGemvMaxRows = 4;
// plan.mt is unused; tiles_per_split counts 32-row tiles
DecodePlan plan_gemv(int64_t M, int64_t K, int64_t N, int64_t group_size);
int launch_gemv(const DecodeParams& p, const DecodePlan& plan, int max_bits, int dtype, bool dense, hipStream_t st);
int launch_sigma(const uint16_t* x, int64_t ldx, int M, int K, int dtype, float* sigma, hipStream_t st);
// The union statistic's grade word of every K row (grade_word: zone set and
// dequantization row constant, for max_bits / 2 planes), K uint32 at grades
int launch_grade_words(const uint16_t* x, int64_t ldx, int M, int K, int dtype, int max_bits,
                       const GradeThresholds& thr, uint32_t* grades, hipStream_t st);

struct PrefillParams {
  const uint16_t* x;
  int64_t ldx;
  const uint32_t* planes;
  const uint16_t* scale;
  const uint16_t* bias;
  uint16_t* y;
  GradeThresholds thr;
  int M, K, N, NW, gs;
  const float* sigma;  // union statistic [K] (graded mode), else nullptr
  int splits;            // grid.z: K ranges (1: y written directly)
  int stages_per_split;  // set by launch_prefill
  float* partial;        // [splits][M][N] fp32 when splits > 1 (the reduce kernel follows)
  uint32_t* counters;    // tall kernel with splits > 1: per split tile, zero on entry
  int dp_tiles;          // tall kernel: tiles computed whole, before the split ones
  const uint32_t* grades;  // tall kernel, graded: grade word of every K row (launch_grade_words)
};

// Prefill path (M > kDecodeMaxRows): dequantize-into-LDS MFMA GEMM.  p.splits
// is an upper bound; *splits_run receives the number of K ranges launched
// (partial sums to reduce when above 1).
int launch_prefill(const PrefillParams& p, int max_bits, int dtype, bool dense, hipStream_t st,
                   int* splits_run);
int prefill_block_rows(int64_t M, int64_t N);
// K ranges of a prefill launch: enough to give every CU a block when the
// (column block, row block) grid alone is smaller, each range at least 256
// rows of K and the partial sums at most kMaxPrefillPartialBytes.  Depends
// only on (M, K, N), so the workspace size does too.
constexpr size_t kMaxPrefillPartialBytes = size_t(256) << 20;
int prefill_splits(int64_t M, int64_t K, int64_t N);

// Large-batch prefill (prefill_tall.hip): (64 * rt) x 128 output tiles over
// four waves (one per SIMD), x repacked into MFMA fragments and loaded
// straight into registers, the weight dequantized per 64-row stage into LDS
// and shared by the block's waves.  From kTallPrefillRows rows (from
// kTallWideRows when the weight has at least kTallWideColBlocks blocks of
// 128 columns), K and the group size multiples of 64, N % 128 == 0 and the
// repacked x below 2^31 bytes.  The first dp_tiles tiles run whole; the
// others (the last, partly filled round) split K into `splits` ranges,
// completed in the kernel (partial sums, per-tile counters).
constexpr int64_t kTallPrefillRows = 256;
// 129-255 rows of a weight this wide fill the GPU with one round of whole
// 256-row tiles, which takes the same time as at 256 rows, while the fused
// kernel's grid then needs two row tiles per column block: Llama-3-8B gate_up
// at 192 / 255 rows took 80.8 / 84.6 us here against 118.2 / 120.9 us fused
// (graded 98.8 against 139.5 / 143.5).  At 80-128 rows, and for the narrower
// weights (down, o_proj at 80-255 rows), the fused kernel stays faster.
constexpr int64_t kTallWideRows = 129;
constexpr int64_t kTallWideColBlocks = 192;
struct TallPlan {
  int rt;        // 16-row tiles per wave: 8 (512-row blocks) or 4 (256-row blocks)
  int splits;    // K ranges of the split tiles
  int dp_tiles;  // tiles computed whole (all when splits == 1)
  int tiles;     // output tiles
};
bool prefill_tall_applies(int64_t M, int64_t K, int64_t N, int64_t ldx, int gs);
// max_partial: bytes available for split-K partial sums
TallPlan plan_tall(int64_t M, int64_t K, int64_t N, size_t max_partial);
inline size_t tall_partial_bytes(const TallPlan& pl, int64_t M, int64_t N) {
  (void)M, (void)N;
  return pl.splits > 1 ? (size_t)(pl.tiles - pl.dp_tiles) * (size_t)pl.splits * (size_t)(64 * pl.rt) * 128 * 4 : 0;
}
// p.x is the repacked copy of the activations (launch_repack_x; p.ldx unused)
int launch_prefill_tall(const PrefillParams& p, const TallPlan& plan, int max_bits, int dtype, bool dense,
                        hipStream_t st);
// x [M][ldx] into the A-fragment order the kernel reads (tall_x_bytes bytes)
size_t tall_x_bytes(int64_t M, int64_t K);
int launch_repack_x(const uint16_t* x, int64_t ldx, int M, int K, uint16_t* xt, hipStream_t st);

// Large-batch fp16 prefill without the library path (prefill_wide.hip):
// 256 x 256 output tiles, the weight dequantized into LDS per 64-row stage.
// From kWidePrefillRows rows, N % 256 == 0, K and the group size multiples of
// 64, (M + 256) * ldx * 2 < 2^31, and at least kWideMinTiles tiles: one block
// per CU, so smaller grids leave CUs idle and the fused kernel's 128-row tiles
// are faster (o_proj at 2048 rows: 128 tiles, 164 against 125 us; qkv: 192
// tiles, 172 against 235 us).
constexpr int64_t kWidePrefillRows = 512;
constexpr int64_t kWideMinTiles = 192;
bool prefill_wide_applies(int64_t M, int64_t K, int64_t N, int64_t ldx, int gs, int dtype);
// one launch over the whole K range (p.splits, p.partial unused)
int launch_prefill_wide(const PrefillParams& p, int max_bits, bool dense, hipStream_t st);

// Prefill from kLibraryGemmRows rows (and N % 64 == 0): the weight Wt[N][K] =
// RNE(w * s) (graded: RNE(w_eff * s) from the union statistic) is written
// once (dequant.hip), then a library GEMM multiplies it (blas.hip); below,
// and for other N, the fused dequantize-into-LDS kernel.  (Dense: at 256 rows
// the fused kernel was faster for all four Llama-3-8B shapes, at 512 slower
// for three of them, at 2048 rows 1.5-1.9x slower; graded: 332 us fused
// against 362 us for the four shapes at 256 rows, 557 against 421 at 512.)
constexpr int64_t kLibraryGemmRows = 512;
// bf16 dequantizes in fp32 in the fused kernel, which makes it slower than in
// fp16 (gate_up at 255 rows: 206 against 113 us): the four shapes took 418 us
// fused and 319-328 us on the library path at 255 rows, 261 against 318 at
// 128, and about even at 192 (where the library GEMM's choice for o_proj and
// down is slow), hence the midpoint
constexpr int64_t kLibraryGemmRowsBf16 = 224;
// Whether a prefill product takes the library path.  Batches of 257-511 rows
// take it too when the fused kernel's grid of 128-row tiles needs more than
// one round of blocks (it is then not split over K, and each round runs the
// whole K: gate_up at 320 rows took 227 us fused, 143 us here), or when K is
// at most kLibraryMaxKMidRows (qkv at 320 / 384 / 448 rows: 55 / 57 / 72 us
// fused, 52 / 52 / 52 here, graded 68 / 70 / 89 against 57 / 60 / 62; o_proj
// 2-16 % faster here).  down (K = 14336) stays fused there (dense 95 / 98 /
// 116 us against 105 / 108 / 121); up to 256 rows the fused kernel is faster
// (qkv at 256 rows: 42 against 58 us).
constexpr int64_t kLibraryMaxKMidRows = 8192;
inline bool use_library_gemm(int64_t M, int64_t K, int64_t N, int dtype) {
  if (N % 64 != 0) return false;
  if (M >= kLibraryGemmRows) return true;
  if (dtype == GRINQH_DTYPE_BF16 && M >= kLibraryGemmRowsBf16) return true;
  return M > 256 && (K <= kLibraryMaxKMidRows || ((N / 16 + 15) / 16) * ((M + 127) / 128) > kTargetBlocks);
}
// Graded fp16 library path: the dense weight RNE(w_eff * s) overflows fp16
// where |w_eff| * |s| > 65504, which the reference's union GEMV (fp32
// products) does not.  The statistic pass also writes, per block of its
// second pass, the largest |scale| (fp16 bits) of a share of the scale array
// (scale_range_slots(K) words); the dequantization takes from them an
// exponent e >= 0 that brings every |w_eff * s * 2^-e| within range, writes
// RNE(w_eff * s * 2^-e) and fills the GEMM's alpha vector (one value per
// output column, read from device memory) with 2^e.  e = 0 (alpha 1) for any
// weight whose scales are below 65504 / 2^(max_bits-1).
inline int scale_range_slots(int64_t K) { return (int)((K + 63) / 64); }
// sigma == nullptr: dense; else graded with the union statistic sigma[K].
// slots / alpha (N floats): the graded fp16 overflow guard (nullptr: none).
int launch_dequant_nk(const uint32_t* planes, const uint16_t* scale, uint16_t* wt, int K, int N, int gs,
                      int max_bits, int dtype, const float* sigma, const GradeThresholds& thr,
                      const uint32_t* slots, float* alpha, hipStream_t st);
// Union statistic of a graded library-path batch in two passes: column
// maxima of row chunks (partial: chunks x K floats), then their maximum
// (sigma: K floats); flags (ceil(K/256) x M bytes) marks the rows holding an
// inf or NaN.  Chunks of at least 32 rows, at most 64 chunks.
inline int sigma_chunk_rows(int64_t M) {
  const int64_t r = ((M + 63) / 64 + 7) / 8 * 8;
  return (int)(r > 32 ? r : 32);
}
// scale != nullptr: also the scale-range slots of the overflow guard over the
// n_scale values of scale
int launch_sigma_chunks(const uint16_t* x, int64_t ldx, int M, int K, int dtype, float* partial, uint8_t* flags,
                        float* sigma, const uint16_t* scale, int64_t n_scale, uint32_t* slots, hipStream_t st);
// y = RNE(y + bias) per row, in the activation dtype (N % 8 == 0, 16-byte
// aligned y and bias): the library GEMM writes its rounded output without
// bias, so that the bias add is a second rounding as in the reference
int launch_add_bias_rows(uint16_t* y, const uint16_t* bias, int64_t M, int N, int dtype, hipStream_t st);
// after the GEMM: the outputs of every flagged row become NaN
int launch_nonfinite_rows_to_nan(const uint8_t* flags, int M, int K, uint16_t* y, int N, int dtype, hipStream_t st);
// y[m][n] = alpha[n] * (x[M][K] @ wt[N][K]^T)[m][n] (+ bias[n]) in the
// activation dtype, fp32 accumulation; alpha = 1, or the N-vector alpha read
// by the GEMM from device memory.  The first call of a shape times the
// library's candidate algorithms; prelude (optional) enqueues on a given
// stream the work that precedes the GEMM in the product (the dequantization
// of wt), run before each timed candidate.
using GemmPrelude = std::function<int(hipStream_t)>;
// Whether the library offers an algorithm without workspace for this GEMM
// (asked once per shape and thread, nothing launched).  It offered none for
// a very deep, narrow product (K = 1048832, N = 64, 512 rows); such products
// take the hand-written prefill kernels (wide-tile or fused).
bool gemm_x_wt_supported(int64_t M, int64_t N, int64_t K, int64_t ldx, int dtype, bool bias, bool alpha_vector);
int gemm_x_wt(const uint16_t* x, int64_t ldx, const uint16_t* wt, const uint16_t* bias, uint16_t* y, int64_t M,
              int64_t N, int64_t K, int dtype, const float* alpha, hipStream_t st,
              const GemmPrelude* prelude = nullptr);


// Benchmark timing of a product's main kernel: when armed (by
// grinqh_time_next_product, for the calling thread's next product), the next
// main-kernel launch on this thread hands the two events to the dispatch
// itself (hipExtLaunchKernelGGL), which records them as the kernel starts and
// ends: their interval is the kernel's execution alone, without the event and
// dispatch overhead that records around the launch would add.
struct KernelTiming {
  hipEvent_t start = nullptr, stop = nullptr;
};
extern thread_local KernelTiming t_kernel_timing;

template <typename P>
inline void launch_main_kernel(void (*kernel)(P), dim3 grid, dim3 block, hipStream_t st, const P& p) {
  KernelTiming& kt = t_kernel_timing;
  if (kt.start != nullptr) {
    hipExtLaunchKernelGGL(kernel, grid, block, 0, st, kt.start, kt.stop, 0, p);
    kt = KernelTiming{};
  } else {
    hipLaunchKernelGGL(kernel, grid, block, 0, st, p);
  }
}

// Producer fusion (producer.hip): rows per chunk of the column maxima the
// producers write, and the producers themselves.
constexpr int kSigmaChunkRows = 16;
int launch_rmsnorm_sigma(const uint16_t* x, int64_t ldx, const uint16_t* residual, uint16_t* residual_out,
                         const uint16_t* weight, float eps, uint16_t* y, float* sigma_chunks, int M, int K, int dtype,
                         hipStream_t st);
int launch_silu_mul_sigma(const uint16_t* gu, int64_t ld, uint16_t* y, float* sigma_chunks, int M, int F, int dtype,
                          hipStream_t st);

// sigma_k of a precomputed statistic: the maximum of its chunk maxima
__device__ __forceinline__ float precomputed_sigma(const DecodeParams& p, int k) {
  float s = p.sigma[k];
  for (int c = 1; c < p.sigma_chunks; ++c) s = fmaxf(s, p.sigma[(int64_t)c * p.K + k]);
  return s;
}

int launch_pack_planes(const uint32_t* U, uint32_t* out, int K, int N, int max_bits, hipStream_t st);
int launch_prepare_weight(const int8_t* W, uint32_t* out, int K, int N, int max_bits, hipStream_t st);
int launch_unpack_planes(const uint32_t* P, const int64_t* rows, uint32_t* out, int n_rows, int N, int Z,
                         hipStream_t st);
int launch_dequant(const uint32_t* P, const uint16_t* scale, void* out, int K, int N, int max_bits, int gs,
                   int dtype, hipStream_t st);
int launch_grade(const uint16_t* x, int64_t ldx, int M, int K, const float* t, int max_bits, int dtype,
                 uint8_t* bits, int32_t* beta, hipStream_t st);

}  // namespace grinqh
