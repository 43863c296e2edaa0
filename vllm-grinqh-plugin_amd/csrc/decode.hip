// Decode-regime GRINQH product (M <= 64 per launch): graded or dense
// y = x * W_eff on v_mfma_f32_16x16x32_{f16,bf16}, HBM-bound.
//
// Replaces the reference's Triton GEMVs grinqh_gemv_uint32_packed
// (grinqh/kernel.py:39-167, one row) and grinqh_gemv_uint32_packed_batch_union
// (:170-360, batch union), and the dense branch of grinqh_gemm_or_gemv for
// small batches (:663-680, semantics of :561-587).
//
// Work decomposition
//   grid.x  = column block: 16 plane-word columns w0..w0+15 = 256 logical
//             columns (16 column tiles r of 16 contiguous columns r*NW + w0 + c)
//   grid.y  = K range of `tiles_per_split` 32-row tiles (split-K)
//   4 waves = MT groups of output dwords j x (4/MT) K sub-ranges
//
// Per 32-row tile each lane (c = lane&15, q = lane>>4) owns rows 8q..8q+7 of
// word column c.  It loads, for every plane z active in a row, one 32-bit
// plane word (predicated per row, so only the planes a row needs are fetched),
// rebuilds the masked code bytes of its 16 columns with rotate+mask, and turns
// row pairs into the MFMA B operand:
//   fp16: 0x64 | byte  -> 1024 + u exactly     (u = offset-binary code)
//   bf16: cvt_f32_ubyte, upper half            -> u exactly
// The constant offset and the midpoint bias beta are removed by one extra MFMA
// per tile whose B operand is the per-row value beta*2^sh - off (a "correction
// column" shared by all 16 columns), so per scale group
//   y += s[g][n] * 2^-sh * (C[m][n] + Cv[m]).
// Scales are applied per 128-row group in fp32 as in grinqh/kernel.py:148-158.
//
// Split-K partials are reduced deterministically: the 4/MT waves of a block
// through LDS in fixed order, the K ranges by the last-arriving block (fixed
// order over ranges), which also applies the output cast and bias.
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

constexpr int kDecodeRowsMax = 8192;  // rows graded per block (LDS: 3 bytes per row)

template <typename DT>
struct BOperand;

// fp16: B = 1024 + u, built as 0x64 in the high byte and the code byte in the low byte.
template <>
struct BOperand<F16> {
  static constexpr float kBase = 1024.f;
  __device__ __forceinline__ static void build(const uint32_t (&V)[8], u32x4_t (&B)[4]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
      const uint32_t lo = perm(V[2 * p + 1], V[2 * p], 0x05010400u);  // a0 b0 a1 b1
      const uint32_t hi = perm(V[2 * p + 1], V[2 * p], 0x07030602u);  // a2 b2 a3 b3
      B[0][p] = perm(0x64646464u, lo, 0x04010400u);
      B[1][p] = perm(0x64646464u, lo, 0x04030402u);
      B[2][p] = perm(0x64646464u, hi, 0x04010400u);
      B[3][p] = perm(0x64646464u, hi, 0x04030402u);
    }
  }
};

// bf16: B = u (0..255 has at most 8 significant bits, exact in bf16).
template <>
struct BOperand<BF16> {
  static constexpr float kBase = 0.f;
  __device__ __forceinline__ static void build(const uint32_t (&V)[8], u32x4_t (&B)[4]) {
#pragma unroll
    for (int p = 0; p < 4; ++p) {
#pragma unroll
      for (int beta = 0; beta < 4; ++beta) {
        const float a = (float)((V[2 * p] >> (8 * beta)) & 0xFFu);
        const float b = (float)((V[2 * p + 1] >> (8 * beta)) & 0xFFu);
        B[beta][p] = perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
      }
    }
  }
};

template <typename DT, int MT, int Z, bool DENSE>
__global__ __launch_bounds__(256, 2) void decode_kernel(DecodeParams p) {
  constexpr int NJ = 4 / MT;   // output dwords j per wave
  constexpr int KW = 4 / MT;   // K sub-ranges per block
  constexpr int SH = 8 - 2 * Z;
  constexpr int NRED = (KW - 1) * MT > 0 ? (KW - 1) * MT : 1;

  __shared__ __align__(16) uint8_t s_bits[kDecodeRowsMax];
  __shared__ __align__(16) uint16_t s_bv[kDecodeRowsMax];
  __shared__ f32x4_t s_red[NRED * 16 * 64];
  __shared__ int s_last;

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int jg = wave % MT, kw = wave / MT;
  const int c = lane & 15, q = lane >> 4;
  const int w0 = blockIdx.x * 16;
  const int split = blockIdx.y;
  const int ntiles_total = p.K >> 5;
  const int tile0 = split * p.tiles_per_split;
  const int tile1 = min(tile0 + p.tiles_per_split, ntiles_total);
  const int nt = tile1 - tile0;
  const int row0 = tile0 * 32;

  // ---- phase 1: grade the block's rows (zone bits + correction-column value)
  for (int rr = tid; rr < nt * 32; rr += 256) {
    const int k = row0 + rr;
    uint32_t bits;
    if (DENSE) {
      bits = (1u << Z) - 1u;
    } else {
      const float s = p.sigma != nullptr ? p.sigma[k] : column_absmax<DT>(p.x, p.ldx, p.M, k);
      bits = zone_bits<Z>(s, p.thr.t);
    }
    s_bits[rr] = (uint8_t)bits;
    const int beta = DENSE ? 0 : midpoint_bias<Z>(bits);
    const float off = BOperand<DT>::kBase + ((bits & 1u) ? 128.f : 0.f);
    s_bv[rr] = from_f32<DT>((float)(beta * (1 << SH)) - off);
  }
  __syncthreads();

  // ---- phase 2: main loop over this wave's tiles, one scale group at a time
  f32x4_t Y[MT][NJ][4];
  f32x4_t C[MT][NJ][4];
  f32x4_t Cv[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int b = 0; b < 4; ++b) Y[mt][jj][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  const bool col_ok = (w0 + c) < p.NW;
  const int wc = col_ok ? (w0 + c) : (p.NW - 1);  // clamped word column: loads stay in bounds
  const int64_t rstride = (int64_t)Z * p.NW;
  const uint32_t* pbase = p.planes + wc;
  const float post = 1.0f / (float)(1 << SH);
  const int t_begin = (nt * kw) / KW, t_end = (nt * (kw + 1)) / KW;
  const int tiles_per_group = p.gs >> 5;
  // rows of the A operand: m = 16*mt + c, clamped so every load is in bounds
  // (rows >= M only feed output rows that are never written)
  const uint16_t* xrow[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt) xrow[mt] = p.x + (int64_t)min(16 * mt + c, p.M - 1) * p.ldx + 8 * q;

  for (int t = t_begin; t < t_end;) {
    const int g = (row0 + 32 * t) / p.gs;
    const int t_stop = min(t_end, (g + 1) * tiles_per_group - tile0);
    // prefetch this group's scales (independent loads, consumed after the tiles)
    uint16_t sraw[NJ][4];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int b = 0; b < 4; ++b)
        sraw[jj][b] = p.scale[(int64_t)g * p.N + (int64_t)(4 * (jg * NJ + jj) + b) * p.NW + wc];
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      Cv[mt] = f32x4_t{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b) C[mt][jj][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    }

    for (; t < t_stop; ++t) {
      const int k0 = row0 + t * 32;
      const int rr = t * 32 + 8 * q;
      const u32x2_t mb = *reinterpret_cast<const u32x2_t*>(&s_bits[rr]);
      const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(&s_bv[rr]);

      uint32_t D[8][Z];
      uint32_t init[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const uint32_t bits = (mb[e >> 2] >> (8 * (e & 3))) & 0xFFu;
        init[e] = (bits & 1u) ? 0x80808080u : 0u;
        const uint32_t* rowp = pbase + (int64_t)(k0 + 8 * q + e) * rstride;
#pragma unroll
        for (int z = 0; z < Z; ++z) {
          D[e][z] = (col_ok && ((bits >> z) & 1u)) ? __builtin_nontemporal_load(rowp + (int64_t)z * p.NW) : 0u;
        }
      }

      u32x4_t A[MT];
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) A[mt] = *reinterpret_cast<const u32x4_t*>(xrow[mt] + k0);

#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        const int j = jg * NJ + jj;
        uint32_t V[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) V[e] = rebuild_dword<Z>(D[e], init[e], j);
        u32x4_t B[4];
        BOperand<DT>::build(V, B);
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) C[mt][jj][b] = mfma16x16x32<DT>(A[mt], B[b], C[mt][jj][b]);
      }
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) Cv[mt] = mfma16x16x32<DT>(A[mt], bv, Cv[mt]);
    }

    // group epilogue: y += s[g][n] * 2^-sh * (C + Cv)
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const float sc = to_f32<DT>(sraw[jj][b]) * post;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int e = 0; e < 4; ++e) Y[mt][jj][b][e] = fmaf(sc, C[mt][jj][b][e] + Cv[mt][e], Y[mt][jj][b][e]);
      }
  }

  // ---- phase 3: reduce the K sub-ranges of this block (fixed order)
  if (KW > 1) {
    if (kw > 0) {
      const int slot = (kw - 1) * MT + jg;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b) s_red[(slot * 16 + (mt * NJ + jj) * 4 + b) * 64 + lane] = Y[mt][jj][b];
    }
    __syncthreads();
    if (kw == 0) {
      for (int k2 = 1; k2 < KW; ++k2) {
        const int slot = (k2 - 1) * MT + jg;
#pragma unroll
        for (int mt = 0; mt < MT; ++mt)
#pragma unroll
          for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
            for (int b = 0; b < 4; ++b) Y[mt][jj][b] += s_red[(slot * 16 + (mt * NJ + jj) * 4 + b) * 64 + lane];
      }
    }
  }

  // ---- phase 4: output (direct, or split-K partials + last-block reduction)
  // Output (m, n) of this lane: m = 16*mt + 4*q + e, n = (4*(jg*NJ+jj)+b)*NW + w0 + c.
  // Loads below use clamped (in-bounds) rows/columns so they carry no branches
  // and issue back to back; only the stores are predicated.
  auto col_of = [&](int jj, int b) -> int64_t { return (int64_t)(4 * (jg * NJ + jj) + b) * p.NW + wc; };
  auto store_final = [&](const f32x4_t (&R)[MT][NJ][4]) {
    uint16_t braw[NJ][4];
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int b = 0; b < 4; ++b) braw[jj][b] = p.bias != nullptr ? p.bias[col_of(jj, b)] : (uint16_t)0;
    if (!col_ok) return;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = 16 * mt + 4 * q + e;
            if (m < p.M) {
              uint16_t v = from_f32<DT>(R[mt][jj][b][e]);
              if (p.bias != nullptr) v = from_f32<DT>(to_f32<DT>(v) + to_f32<DT>(braw[jj][b]));
              p.y[(int64_t)m * p.N + col_of(jj, b)] = v;
            }
          }
  };

  if (p.splits == 1) {
    if (kw == 0) store_final(Y);
    return;
  }

  if (kw == 0 && col_ok) {
    float* part = p.partial + (int64_t)split * p.M * p.N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = 16 * mt + 4 * q + e;
            if (m < p.M) part[(int64_t)m * p.N + col_of(jj, b)] = Y[mt][jj][b][e];
          }
  }
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = atomicAdd(&p.counters[blockIdx.x], 1u);
    s_last = (prev == (unsigned)(p.splits - 1)) ? 1 : 0;
  }
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (kw == 0) {
    // sum the K ranges in fixed order 0..splits-1 (independent of arrival order)
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b) Y[mt][jj][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};
    for (int s2 = 0; s2 < p.splits; ++s2) {
      const float* part = p.partial + (int64_t)s2 * p.M * p.N;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt)
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int m = min(16 * mt + 4 * q + e, p.M - 1);
              Y[mt][jj][b][e] += part[(int64_t)m * p.N + col_of(jj, b)];
            }
    }
    store_final(Y);
  }
  if (tid == 0) p.counters[blockIdx.x] = 0u;
}

// sigma_k = max_m |x[m][k]| over the whole batch (NaN ignored unless all NaN),
// for launches that split a batch into several decode calls.
template <typename DT>
__global__ __launch_bounds__(256) void sigma_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M, int K,
                                                    float* __restrict__ sigma) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= K) return;
  sigma[k] = column_absmax<DT>(x, ldx, M, k);
}

DecodePlan plan_decode(int64_t M, int64_t K, int64_t N) {
  DecodePlan pl{};
  pl.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int64_t NW = N / 16;
  pl.col_blocks = (int)((NW + 15) / 16);
  const int64_t T = K / 32;
  const int kw = 4 / pl.mt;
  const int64_t tiles_max = kDecodeRowsMax / 32;
  const int64_t min_splits = (T + tiles_max - 1) / tiles_max;
  const int64_t want = (512 + pl.col_blocks - 1) / pl.col_blocks;
  int64_t max_splits = T / (2 * kw);
  if (max_splits < 1) max_splits = 1;
  int64_t splits = want < max_splits ? want : max_splits;
  if (splits < min_splits) splits = min_splits;
  const int64_t bytes_per_split = M * N * (int64_t)sizeof(float);
  if (splits > 1 && bytes_per_split > 0) {
    int64_t cap = (int64_t)kMaxPartialBytes / bytes_per_split;
    if (cap < min_splits) cap = min_splits;
    if (splits > cap) splits = cap;
  }
  if (splits < 1) splits = 1;
  int64_t tps = (T + splits - 1) / splits;
  if (tps < 1) tps = 1;
  splits = (T + tps - 1) / tps;
  if (splits < 1) splits = 1;
  pl.splits = (int)splits;
  pl.tiles_per_split = (int)tps;
  pl.workspace = splits > 1 ? kCounterBytes + (size_t)(splits * bytes_per_split) : 0;
  return pl;
}

template <typename DT, int MT, int Z>
static void launch_decode_t(const DecodeParams& p, const DecodePlan& pl, bool dense, hipStream_t st) {
  const dim3 grid(pl.col_blocks, pl.splits);
  if (dense)
    hipLaunchKernelGGL((decode_kernel<DT, MT, Z, true>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((decode_kernel<DT, MT, Z, false>), grid, dim3(256), 0, st, p);
}

template <typename DT, int MT>
static int launch_decode_mt(const DecodeParams& p, const DecodePlan& pl, int Z, bool dense, hipStream_t st) {
  switch (Z) {
    case 1: launch_decode_t<DT, MT, 1>(p, pl, dense, st); break;
    case 2: launch_decode_t<DT, MT, 2>(p, pl, dense, st); break;
    case 3: launch_decode_t<DT, MT, 3>(p, pl, dense, st); break;
    case 4: launch_decode_t<DT, MT, 4>(p, pl, dense, st); break;
    default: return GRINQH_ERR_INVALID;
  }
  return GRINQH_OK;
}

template <typename DT>
static int launch_decode_dt(const DecodeParams& p, const DecodePlan& pl, int Z, bool dense, hipStream_t st) {
  switch (pl.mt) {
    case 1: return launch_decode_mt<DT, 1>(p, pl, Z, dense, st);
    case 2: return launch_decode_mt<DT, 2>(p, pl, Z, dense, st);
    case 4: return launch_decode_mt<DT, 4>(p, pl, Z, dense, st);
    default: return GRINQH_ERR_INVALID;
  }
}

int launch_decode(const DecodeParams& p, const DecodePlan& pl, int max_bits, int dtype, bool dense,
                  hipStream_t st) {
  const int Z = max_bits / 2;
  const int rc = dtype == GRINQH_DTYPE_BF16 ? launch_decode_dt<BF16>(p, pl, Z, dense, st)
                                            : launch_decode_dt<F16>(p, pl, Z, dense, st);
  if (rc != GRINQH_OK) return rc;
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_sigma(const uint16_t* x, int64_t ldx, int M, int K, int dtype, float* sigma, hipStream_t st) {
  if (K == 0) return GRINQH_OK;
  const dim3 grid((K + 255) / 256);
  if (dtype == GRINQH_DTYPE_BF16)
    hipLaunchKernelGGL(sigma_kernel<BF16>, grid, dim3(256), 0, st, x, ldx, M, K, sigma);
  else
    hipLaunchKernelGGL(sigma_kernel<F16>, grid, dim3(256), 0, st, x, ldx, M, K, sigma);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
