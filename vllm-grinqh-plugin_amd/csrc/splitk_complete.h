// In-kernel split-K completion for the GEMV and decode kernels.
//
// Every K range (split) of a column block stores its fp32 partial sums to
// partial[split][m][n] and then counts itself done on the column block's
// counter.  The range that arrives last adds the partial sums of all ranges in
// range order 0, 1, ..., splits-1 (so the result does not depend on which
// range finished last), casts, adds the bias, writes y and clears the counter
// for the next call.  This replaces a second reduction launch, whose fixed
// cost is comparable to a whole small product.
//
// Memory ordering without cache maintenance: partial sums are stored with
// agent-scope (sc1) stores, which write through the XCD's L2, and every wave
// waits for its stores to complete before the block's counter increment; the
// last block reads them with agent-scope (sc1) loads, which do not hit stale
// L2 lines.  (A __threadfence per block would write back and invalidate the
// whole L2 and costs more than the reduction itself.)  Counters are only
// touched by atomics.  No block waits for another: every block exits after
// its own work.
#pragma once
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

constexpr int kCpolSc1 = 16;  // buffer cache policy: agent scope (sc1)

// Agent-scope store of one partial sum (global_store ... sc1).
__device__ __forceinline__ void store_partial(float* dst, float v) {
  __hip_atomic_store(dst, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Columns of one column block: r * NW + w0 + [0, width) for column tiles
// r = 0..15, clipped at NW (NW % 4 == 0, so a 4-column chunk is either wholly
// inside or wholly outside).  NCK = 4-column chunks per thread (the block's
// M * 16 * width / 4 chunks over the block's NT threads, rounded up).
template <typename DT, int NCK, int NT = 256>
__device__ __forceinline__ void splitk_complete(const DecodeParams& p, int cb, int w0, int width) {
  constexpr int SB = 16 / NCK;  // K ranges per round: 16 loads in flight per thread
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
  __syncthreads();
  if (threadIdx.x == 0) s_last = atomicAdd(&p.counters[cb], 1u) == (unsigned)(p.splits - 1);
  __syncthreads();
  if (!s_last) return;

  const int cpr = width >> 2;  // chunks per column tile
  const int per_m = 16 * cpr;
  const int total = p.M * per_m;
  const uint32_t slab = (uint32_t)p.M * (uint32_t)p.N * 4u;  // bytes per K range (< 2^31 by plan)
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
      p.partial, (short)0, (int)(slab * (uint32_t)p.splits), 0x00020000);

  uint32_t off[NCK];  // byte offset of the chunk in a K range's slab; bit 31: none (reads 0)
  int col[NCK];       // first output column of the chunk
#pragma unroll
  for (int k = 0; k < NCK; ++k) {
    const int i = threadIdx.x + NT * k;
    const int m = i / per_m, rem = i - m * per_m;
    const int r = rem / cpr;
    const int wcol = w0 + 4 * (rem - r * cpr);
    const bool ok = i < total && wcol < p.NW;
    col[k] = r * p.NW + wcol;
    off[k] = ok ? ((uint32_t)m * (uint32_t)p.N + (uint32_t)col[k]) * 4u : 0x80000000u;
  }
  f32x4_t acc[NCK];
#pragma unroll
  for (int k = 0; k < NCK; ++k) acc[k] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < p.splits; s0 += SB) {
    f32x4_t v[NCK][SB];
#pragma unroll
    for (int k = 0; k < NCK; ++k)
#pragma unroll
      for (int ss = 0; ss < SB; ++ss) {
        const bool live = s0 + ss < p.splits && off[k] != 0x80000000u;
        const uint32_t o = live ? off[k] + (uint32_t)(s0 + ss) * slab : 0x80000000u;
        v[k][ss] = __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)o, 0, kCpolSc1));
      }
#pragma unroll
    for (int k = 0; k < NCK; ++k)
#pragma unroll
      for (int ss = 0; ss < SB; ++ss) acc[k] += v[k][ss];
  }
#pragma unroll
  for (int k = 0; k < NCK; ++k) {
    if (off[k] == 0x80000000u) continue;
    const int n = col[k];
    u32x2_t h;
    h[0] = (uint32_t)finish_output<DT>(acc[k][0], p.bias, n) | ((uint32_t)finish_output<DT>(acc[k][1], p.bias, n + 1) << 16);
    h[1] = (uint32_t)finish_output<DT>(acc[k][2], p.bias, n + 2) | ((uint32_t)finish_output<DT>(acc[k][3], p.bias, n + 3) << 16);
    *reinterpret_cast<u32x2_t*>(p.y + (off[k] >> 2)) = h;
  }
  if (threadIdx.x == 0) atomicExch(&p.counters[cb], 0u);
}

}  // namespace grinqh
