// Grade-grouped K order for the graded prefill.
//
// The graded (union) prefill rebuilds each 32-row stage of the weight from the
// planes its rows need.  Rows of one scale group are independent terms of the
// dot product, so they may be consumed in any order: ordering them by zone set
// (stable within a set) makes most stages single-precision, and a stage then
// loads and merges only the planes of its zone set (the OR of its rows' sets)
// instead of all max_bits/2 planes.  The scale of a row depends only on its
// group, and rows never leave their group, so the epilogue is unchanged.
//
//   grade_order_kernel: per scale group, perm[k'] = natural row at sorted
//     position k' (counting sort by zone set over 2^Z keys, stable by row),
//     and stage_bits[k'/32] = OR of the zone sets of the stage's 32 rows.
//   permute_cols_kernel: x_sorted[m][k'] = x[m][perm[k']], so the prefill
//     still reads x with 16-byte loads of 8 consecutive columns.
//
// The grading itself is the same zone_bits() the product uses (S6), applied
// to the batch statistic sigma.
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

// One wave per scale group [k0, k1).
template <int Z>
__global__ __launch_bounds__(64) void grade_order_kernel(const float* __restrict__ sigma, GradeThresholds thr, int K,
                                                         int gs, int* __restrict__ perm,
                                                         uint32_t* __restrict__ stage_bits) {
  constexpr int NKEY = 1 << Z;
  const int lane = threadIdx.x;
  const int k0 = blockIdx.x * gs;
  const int k1 = min(k0 + gs, K);
  const uint64_t below = (1ull << lane) - 1ull;

  // pass 1: rows per zone set
  int cnt[NKEY];
#pragma unroll
  for (int v = 0; v < NKEY; ++v) cnt[v] = 0;
  for (int base = k0; base < k1; base += 64) {
    const int k = base + lane;
    const int key = k < k1 ? (int)zone_bits<Z>(sigma[k], thr.t) : NKEY;
#pragma unroll
    for (int v = 0; v < NKEY; ++v) cnt[v] += __popcll(__ballot(key == v));
  }
  int next[NKEY];  // next sorted position of each zone set
  int acc = 0;
#pragma unroll
  for (int v = 0; v < NKEY; ++v) {
    next[v] = acc;
    acc += cnt[v];
  }

  // pass 2: stable positions
  for (int base = k0; base < k1; base += 64) {
    const int k = base + lane;
    const int key = k < k1 ? (int)zone_bits<Z>(sigma[k], thr.t) : NKEY;
    int pos = 0;
#pragma unroll
    for (int v = 0; v < NKEY; ++v) {
      const uint64_t m = __ballot(key == v);
      if (key == v) pos = next[v] + __popcll(m & below);
      next[v] += __popcll(m);
    }
    if (k < k1) perm[k0 + pos] = k;
  }
  __syncthreads();

  // pass 3: zone-set union of every 32-row stage (stages never straddle a group)
  for (int base = k0; base < k1; base += 64) {
    const int pos = base + lane;
    uint32_t bits = pos < k1 ? zone_bits<Z>(sigma[perm[pos]], thr.t) : 0u;
#pragma unroll
    for (int o = 16; o >= 1; o >>= 1) bits |= (uint32_t)__shfl_xor((int)bits, o);
    if ((lane & 31) == 0 && pos < k1) stage_bits[pos >> 5] = bits;
  }
}

// x_sorted[m][k'] = x[m][perm[k']]; one thread per 8 consecutive sorted columns.
__global__ __launch_bounds__(256) void permute_cols_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                           const int* __restrict__ perm, int M, int K,
                                                           uint16_t* __restrict__ xs) {
  const int chunks = K >> 3;
  const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
  if (idx >= (int64_t)M * chunks) return;
  const int m = (int)(idx / chunks), c = (int)(idx % chunks);
  const int* pc = perm + 8 * c;
  const uint16_t* xr = x + (int64_t)m * ldx;
  u32x4_t v;
#pragma unroll
  for (int i = 0; i < 4; ++i) v[i] = (uint32_t)xr[pc[2 * i]] | ((uint32_t)xr[pc[2 * i + 1]] << 16);
  *reinterpret_cast<u32x4_t*>(xs + (int64_t)m * K + 8 * c) = v;
}

int launch_grade_order(const float* sigma, const GradeThresholds& thr, int K, int gs, int max_bits, int* perm,
                       uint32_t* stage_bits, hipStream_t st) {
  const dim3 grid((K + gs - 1) / gs);
  switch (max_bits / 2) {
    case 1: hipLaunchKernelGGL(grade_order_kernel<1>, grid, dim3(64), 0, st, sigma, thr, K, gs, perm, stage_bits); break;
    case 2: hipLaunchKernelGGL(grade_order_kernel<2>, grid, dim3(64), 0, st, sigma, thr, K, gs, perm, stage_bits); break;
    case 3: hipLaunchKernelGGL(grade_order_kernel<3>, grid, dim3(64), 0, st, sigma, thr, K, gs, perm, stage_bits); break;
    case 4: hipLaunchKernelGGL(grade_order_kernel<4>, grid, dim3(64), 0, st, sigma, thr, K, gs, perm, stage_bits); break;
    default: return GRINQH_ERR_INVALID;
  }
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_permute_cols(const uint16_t* x, int64_t ldx, const int* perm, int M, int K, uint16_t* xs,
                        hipStream_t st) {
  const int64_t threads = (int64_t)M * (K / 8);
  if (threads == 0) return GRINQH_OK;
  const dim3 grid((unsigned)((threads + 255) / 256));
  hipLaunchKernelGGL(permute_cols_kernel, grid, dim3(256), 0, st, x, ldx, perm, M, K, xs);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
