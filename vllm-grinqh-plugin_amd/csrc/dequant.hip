// Dense weight of a large prefill: Wt[n][k] = RNE(w[k][n] * s[k/gs][n]) in the
// activation dtype, stored K-contiguous ([N][K]), for the library GEMM that
// follows (blas.hip).  Graded (union) batches write RNE(w_eff * s) instead,
// with each row's zone set from sigma_k = max_m |x[m][k]|: the planes of its
// inactive zones are masked to zero and its midpoint bias is added, as in the
// fused prefill kernel.  (Every plane is fetched: skipping the inactive ones
// put a sigma load in front of each plane load, and with the 2-byte weight
// write dominating the traffic that made the graded pass 15 % slower than
// the dense one.)
//
// Replaces the dequantization half of grinqh_prefill_gemm_compiled
// (grinqh/kernel.py:571-586: unpack_pyt, sign extension, postshuffle, then
// W * s, compiled torch passes over int8 and fp16 copies of the weight).  The
// values are the same
// RNE(w * s) the fused prefill kernel writes into LDS (Dequant<DT, SH>), so
// both prefill paths multiply the same weight.
//
// HBM-bound: per weight b/8 bytes of planes in, 2 bytes out (plus 2/gs bytes
// of scales).  A block covers 64 rows of K and 32 plane-word columns: it
// loads the tile's plane words as whole 128-byte row segments (16 bytes per
// lane, so N / 16 must be a multiple of 4) into LDS, transposed to [column][k]
// [zone].  Then one lane owns one column c and 8 consecutive rows: it reads its
// 8 x Z words with 16-byte LDS reads and writes, for each of the word's 16
// logical columns n = (4j + beta) * NW + c, one 16-byte run Wt[n][k0 .. k0+8).
// The 8 lanes that share c cover the block's 64 rows, so each store
// instruction writes 8 whole 128-byte lines.  Loading the planes straight
// from HBM in the lanes' own pattern (8 rows x 32 bytes per instruction) ran
// at 3 TB/s, this form at 5 TB/s.
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

namespace {

struct DequantParams {
  const uint32_t* planes;
  const uint16_t* scale;
  uint16_t* wt;        // [N][K]
  const float* sigma;  // graded: union statistic [K]
  GradeThresholds thr;
  int K, N, NW, gs;
  const uint32_t* slots;  // graded fp16: scale-range slots (overflow guard), else nullptr
  int n_slots;
  float* alpha;           // the GEMM's alpha vector [N] when slots != nullptr
};

constexpr int kDqColsPerBlock = 32;  // plane-word columns per block (4 waves x 8)
constexpr int kDqRowsPerBlock = 64;  // rows of K per block

template <typename DT, int Z, bool DENSE>
__global__ __launch_bounds__(256) void dequant_nk_kernel(DequantParams p) {
  constexpr int SH = 8 - 2 * Z;
  constexpr int LROW = 64 * Z + 4;  // words per word column in LDS (16-byte aligned rows)
  __shared__ __align__(16) uint32_t lds[32 * LROW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cb0 = blockIdx.x * kDqColsPerBlock, kb = blockIdx.y * kDqRowsPerBlock;
  // overflow guard (graded fp16): the largest |scale| over the slots
  constexpr bool GUARD = !DENSE && DT::id == F16::id;
  constexpr uint32_t kScaleLimit = 0x7BFFu - ((uint32_t)(2 * Z - 1) << 10);  // 65504 / 2^(2Z-1), fp16 bits
  __shared__ uint32_t s_wmax[4];
  if constexpr (GUARD) {
    uint32_t hm = 0;
    if (p.slots != nullptr)
      for (int i = threadIdx.x; i < p.n_slots; i += 256) hm = max(hm, p.slots[i]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) hm = max(hm, (uint32_t)__shfl_xor((int)hm, o, 64));
    if (lane == 0) s_wmax[wave] = hm;
  }
  {  // NW % 4 == 0: a 4-word piece is wholly inside or outside the row
    const int pc = threadIdx.x & 7;  // 4-word piece of the block's 32 columns
#pragma unroll
    for (int i = 0; i < 2 * Z; ++i) {
      const int seg = (threadIdx.x >> 3) + 32 * i;  // (k, z) of the block tile
      const int k = seg / Z, z = seg % Z;
      u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
      if (kb + k < p.K && cb0 + 4 * pc < p.NW)
        v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p.planes + (int64_t)(kb + k) * Z * p.NW +
                                                                        (int64_t)z * p.NW + cb0 + 4 * pc));
#pragma unroll
      for (int q = 0; q < 4; ++q) lds[(4 * pc + q) * LROW + seg] = v[q];
    }
  }
  __syncthreads();
  int up_exp = 0;  // the weight is written times 2^-up_exp and the GEMM's alpha is 2^up_exp
  if constexpr (GUARD) {
    const uint32_t hm = max(max(s_wmax[0], s_wmax[1]), max(s_wmax[2], s_wmax[3]));
    if (hm > kScaleLimit) up_exp = (int)(hm >> 10) - (int)(kScaleLimit >> 10);
    if (p.alpha != nullptr && blockIdx.y == 0) {  // the block's 16 x 32 output columns
      const float a = __builtin_ldexpf(1.f, up_exp);
      for (int i = threadIdx.x; i < 16 * kDqColsPerBlock; i += 256) {
        const int wcol = cb0 + i % kDqColsPerBlock;
        if (wcol < p.NW) p.alpha[(int64_t)(i / kDqColsPerBlock) * p.NW + wcol] = a;
      }
    }
  }
  const int c = cb0 + wave * 8 + (lane >> 3);
  const int k0 = kb + 8 * (lane & 7);
  if (c >= p.NW || k0 >= p.K) return;  // K % 32 == 0: a run of 8 rows is whole
  uint32_t D[8][Z];
  {
    const uint32_t* l = &lds[(wave * 8 + (lane >> 3)) * LROW + 8 * (lane & 7) * Z];
#pragma unroll
    for (int i = 0; i < 2 * Z; ++i) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(l + 4 * i);
#pragma unroll
      for (int q = 0; q < 4; ++q) D[(4 * i + q) / Z][(4 * i + q) % Z] = v[q];
    }
  }

  const uint16_t* srow = p.scale + (int64_t)(k0 / p.gs) * p.N + c;  // gs % 32 == 0: one group per run
  uint16_t sraw[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) sraw[r] = srow[(int64_t)r * p.NW];
  if (GUARD && up_exp > 0) {
    const float down = __builtin_ldexpf(1.f, -up_exp);
#pragma unroll
    for (int r = 0; r < 16; ++r) sraw[r] = from_f32<DT>(to_f32<DT>(sraw[r]) * down);
  }

  int beta[8];  // midpoint bias of each row's zone set (0: every zone active)
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    if constexpr (!DENSE) {  // graded: inactive planes masked to zero
      const uint32_t bits = zone_bits<Z>(p.sigma[k0 + e], p.thr.t);
      beta[e] = midpoint_bias<Z>(bits);
#pragma unroll
      for (int z = 0; z < Z; ++z) D[e][z] &= 0u - ((bits >> z) & 1u);
    } else {
      beta[e] = 0;
    }
    D[e][0] ^= 0xAAAAAAAAu;  // offset binary: u = int8(U & mask) + 128
#pragma unroll
    for (int z = 1; z < Z; ++z) D[e][z] = rotr(D[e][z], (uint32_t)(2 * z));
  }

  uint16_t* dst = p.wt + (int64_t)c * p.K + k0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t out[4][4];  // [beta][pair]
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      // u - c_row = w_eff * 2^SH for the pair's two rows
      const uint16_t c0 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[2 * pp]));
      const uint16_t c1 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[2 * pp + 1]));
      const uint32_t negc = (uint32_t)c0 | ((uint32_t)c1 << 16);
      const float cb0 = (float)(128 - beta[2 * pp] * (1 << SH)), cb1 = (float)(128 - beta[2 * pp + 1] * (1 << SH));
      uint32_t V[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        const int ee = 2 * pp + e;
        uint32_t h = (Z == 4) ? D[ee][3] : (D[ee][0] & (0x03030303u << (2 * ((3 - j) & 3))));
#pragma unroll
        for (int z = (Z == 4 ? 0 : 1); z < (Z == 4 ? 3 : Z); ++z)
          h = bfi(0x03030303u << (2 * ((3 - z - j) & 3)), D[ee][z], h);
        V[e] = rotr(h, (uint32_t)(32 - 2 * j) & 31u);
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint16_t s = sraw[4 * j + b];
        if constexpr (DT::id == F16::id) {
          out[b][pp] = Dequant<F16, SH>::pair(V[0], V[1], b, negc, (uint32_t)s | ((uint32_t)s << 16));
        } else {
          const float sf = to_f32<DT>(s) * (1.0f / (float)(1 << SH));
          out[b][pp] = Dequant<BF16, SH>::pair_bf16(V[0], V[1], b, cb0, cb1, sf);
        }
      }
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t n = (int64_t)(4 * j + b) * p.NW;
      *reinterpret_cast<u32x4_t*>(dst + n * p.K) = u32x4_t{out[b][0], out[b][1], out[b][2], out[b][3]};
    }
  }
}

// Union statistic of a large graded batch, first pass: a block takes 256
// columns (8 per lane, 16-byte loads) of a chunk of rows, 8 rows at a time,
// and writes its column maxima to partial[chunk][k] (NaN ignored unless every
// value is NaN, as fmaxf does).  It also records, per row, whether the row's
// 256 values hold an inf or NaN: flags[column block][m].
template <typename DT>
__global__ __launch_bounds__(256) void sigma_chunks_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M, int K,
                                                           int rows_per_chunk, float* __restrict__ partial,
                                                           uint8_t* __restrict__ flags) {
  constexpr uint32_t EXP = DT::id == F16::id ? 0x7C00u : 0x7F80u;  // all-ones exponent: inf or NaN
  __shared__ float s_part[8][256 + 4];
  const int l = threadIdx.x & 31, g = threadIdx.x >> 5;
  const int k = blockIdx.x * 256 + 8 * l;
  const bool col_ok = k < K;  // K % 8 == 0: a lane's 8 columns are all in or all out
  const int r0 = blockIdx.y * rows_per_chunk, r1 = min(r0 + rows_per_chunk, M);
  float s[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) s[i] = __int_as_float(0x7fc00000);  // NaN: no row seen yet
  for (int mb = r0 + g; mb < r1; mb += 32) {  // 4 rows' loads in flight
    u32x4_t v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = mb + 8 * j;
      v[j] = u32x4_t{0u, 0u, 0u, 0u};
      if (col_ok && m < r1) v[j] = *reinterpret_cast<const u32x4_t*>(x + (int64_t)m * ldx + k);  // ldx % 8 == 0
    }
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int m = mb + 8 * j;
      if (m >= r1) break;  // the same for the 32 lanes of a row
      bool bad = false;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const uint16_t lo = (uint16_t)(v[j][q] & 0xFFFFu), hi = (uint16_t)(v[j][q] >> 16);
        s[2 * q] = fmaxf(s[2 * q], fabsf(to_f32<DT>(lo)));
        s[2 * q + 1] = fmaxf(s[2 * q + 1], fabsf(to_f32<DT>(hi)));
        bad |= ((lo & EXP) == EXP) | ((hi & EXP) == EXP);
      }
      // the 32 lanes of this half-wave share row m (lanes of a finished half read as 0)
      const uint64_t bal = __ballot(bad);
      if (l == 0) flags[(int64_t)blockIdx.x * M + m] = ((bal >> (threadIdx.x & 32)) & 0xFFFFFFFFull) != 0;
    }
  }
#pragma unroll
  for (int i = 0; i < 8; ++i) s_part[g][8 * l + i] = s[i];
  __syncthreads();
  const int kk = blockIdx.x * 256 + threadIdx.x;
  if (kk < K) {
    float r = s_part[0][threadIdx.x];
#pragma unroll
    for (int gg = 1; gg < 8; ++gg) r = fmaxf(r, s_part[gg][threadIdx.x]);
    partial[(int64_t)blockIdx.y * K + kk] = r;
  }
}

// Second pass: sigma[k] = fmaxf over the chunks' maxima (exact in any order).
// A block takes 64 columns; its 4 waves take every 4th chunk, all of a wave's
// loads (16 for the at most 64 chunks) in flight at once, and combine through
// LDS.
// With slots != nullptr, block b also writes slots[b] = the largest |value|
// (fp16 bits) of its share of the n_scale scales (the overflow guard of the
// graded fp16 dequantization), scanned while the chunk loads are in flight.
__global__ __launch_bounds__(256) void sigma_chunks_reduce_kernel(const float* __restrict__ partial, int chunks,
                                                                  int K, float* __restrict__ sigma,
                                                                  const uint16_t* __restrict__ scale,
                                                                  int64_t n_scale, uint32_t* __restrict__ slots) {
  constexpr int BATCH = 16;
  __shared__ float s_part[4][64];
  __shared__ uint32_t s_smax[4];
  const int cl = threadIdx.x & 63, cg = threadIdx.x >> 6;
  const int k = blockIdx.x * 64 + cl;
  const int kc = min(k, K - 1);  // columns past the end read a valid one and are not stored
  // every load is issued (chunks past the end repeat the last one, which the
  // maximum absorbs): a load under a condition was waited for at once
  float v[BATCH];
#pragma unroll
  for (int j = 0; j < BATCH; ++j) v[j] = partial[(int64_t)min(cg + 4 * j, chunks - 1) * K + kc];
  if (slots != nullptr) {
    // each block's share of the scales (whole 16-byte vectors when the
    // array is 16-byte aligned), eight vectors per thread in flight
    const int64_t per = ((n_scale + gridDim.x - 1) / gridDim.x + 7) & ~(int64_t)7;
    const int64_t i0 = min((int64_t)blockIdx.x * per, n_scale), i1 = min(i0 + per, n_scale);
    uint32_t hm = 0;
    int64_t tail = i0;
    if ((reinterpret_cast<uintptr_t>(scale) & 15u) == 0) {
      const int64_t nv = (i1 - i0) / 8;
      const u32x4_t* sv = reinterpret_cast<const u32x4_t*>(scale + i0);
      for (int64_t j = threadIdx.x; j < nv; j += 8 * 256) {
        u32x4_t w[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) w[u] = j + 256 * u < nv ? sv[j + 256 * u] : u32x4_t{0u, 0u, 0u, 0u};
#pragma unroll
        for (int u = 0; u < 8; ++u)
#pragma unroll
          for (int q = 0; q < 4; ++q) hm = max(hm, max(w[u][q] & 0x7FFFu, (w[u][q] >> 16) & 0x7FFFu));
      }
      tail = i0 + 8 * nv;
    }
    for (int64_t i = tail + threadIdx.x; i < i1; i += 256) hm = max(hm, (uint32_t)scale[i] & 0x7FFFu);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) hm = max(hm, (uint32_t)__shfl_xor((int)hm, o, 64));
    if (cl == 0) s_smax[cg] = hm;
  }
  float s = v[0];
#pragma unroll
  for (int j = 1; j < BATCH; ++j) s = fmaxf(s, v[j]);
  for (int c0 = cg + 4 * BATCH; c0 < chunks; c0 += 4 * BATCH) {  // more than 64 chunks: further rounds
#pragma unroll
    for (int j = 0; j < BATCH; ++j) v[j] = partial[(int64_t)min(c0 + 4 * j, chunks - 1) * K + kc];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) s = fmaxf(s, v[j]);
  }
  s_part[cg][cl] = s;
  __syncthreads();
  if (cg == 0 && k < K) sigma[k] = fmaxf(fmaxf(s_part[0][cl], s_part[1][cl]), fmaxf(s_part[2][cl], s_part[3][cl]));
  if (slots != nullptr && threadIdx.x == 0) slots[blockIdx.x] = max(max(s_smax[0], s_smax[1]), max(s_smax[2], s_smax[3]));
}

// Graded products: a row of x holding a non-finite value has every output
// non-finite, and the graded kernels return those outputs as NaN (see
// graded_nonfinite_to_nan); the library GEMM leaves inf where the fused
// kernels give NaN, so this pass (one block per row, after the GEMM) writes
// NaN over the outputs of every row that the statistic pass flagged.
__global__ __launch_bounds__(256) void nonfinite_rows_to_nan_kernel(const uint8_t* __restrict__ flags, int col_blocks,
                                                                    int M, uint16_t* __restrict__ y, int N,
                                                                    uint16_t nan) {
  const int m = blockIdx.x;
  int bad = 0;
  for (int i = threadIdx.x; i < col_blocks; i += 256) bad |= flags[(int64_t)i * M + m];
  if (!__syncthreads_or(bad)) return;
  for (int n = threadIdx.x; n < N; n += 256) y[(int64_t)m * N + n] = nan;
}

// y[m][n] = RNE(y[m][n] + bias[n]) in the activation dtype: the bias add of
// the reference (y.add_(bias) on the matmul's rounded output,
// grinqh/kernel.py:706-708) after a GEMM that wrote y without bias.  One
// thread per 8 columns (N % 8 == 0, 16-byte aligned rows).
template <typename DT>
__global__ __launch_bounds__(256) void add_bias_rows_kernel(uint16_t* __restrict__ y, const uint16_t* __restrict__ bias,
                                                            int64_t M, int N) {
  const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;  // 8-column chunk
  const int cpr = N / 8;
  if (i >= M * cpr) return;
  const int64_t m = i / cpr;
  const int n0 = (int)(i - m * cpr) * 8;
  u32x4_t v = *reinterpret_cast<const u32x4_t*>(&y[m * N + n0]);
  const u32x4_t b = *reinterpret_cast<const u32x4_t*>(&bias[n0]);
#pragma unroll
  for (int h = 0; h < 4; ++h) {
    const float a0 = to_f32<DT>((uint16_t)(v[h] & 0xFFFFu)) + to_f32<DT>((uint16_t)(b[h] & 0xFFFFu));
    const float a1 = to_f32<DT>((uint16_t)(v[h] >> 16)) + to_f32<DT>((uint16_t)(b[h] >> 16));
    v[h] = (uint32_t)from_f32<DT>(a0) | ((uint32_t)from_f32<DT>(a1) << 16);
  }
  *reinterpret_cast<u32x4_t*>(&y[m * N + n0]) = v;
}

template <typename DT, bool DENSE>
int launch_dequant_dt(const DequantParams& p, int max_bits, hipStream_t st) {
  const dim3 grid((unsigned)((p.NW + kDqColsPerBlock - 1) / kDqColsPerBlock),
                  (unsigned)((p.K + kDqRowsPerBlock - 1) / kDqRowsPerBlock));
  switch (max_bits) {
    case 2: launch_main_kernel(dequant_nk_kernel<DT, 1, DENSE>, grid, dim3(256), st, p); break;
    case 4: launch_main_kernel(dequant_nk_kernel<DT, 2, DENSE>, grid, dim3(256), st, p); break;
    case 6: launch_main_kernel(dequant_nk_kernel<DT, 3, DENSE>, grid, dim3(256), st, p); break;
    case 8: launch_main_kernel(dequant_nk_kernel<DT, 4, DENSE>, grid, dim3(256), st, p); break;
    default: return GRINQH_ERR_INVALID;
  }
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace

int launch_dequant_nk(const uint32_t* planes, const uint16_t* scale, uint16_t* wt, int K, int N, int gs,
                      int max_bits, int dtype, const float* sigma, const GradeThresholds& thr,
                      const uint32_t* slots, float* alpha, hipStream_t st) {
  if (K % 32 != 0 || N % 64 != 0 || gs % 32 != 0 || (int64_t)K * N >= ((int64_t)1 << 40)) return GRINQH_ERR_INVALID;
  const DequantParams p{planes, scale, wt, sigma, thr, K, N, N / 16, gs, slots, scale_range_slots(K), alpha};
  const bool bf16 = dtype == GRINQH_DTYPE_BF16;
  if (sigma == nullptr)
    return bf16 ? launch_dequant_dt<BF16, true>(p, max_bits, st) : launch_dequant_dt<F16, true>(p, max_bits, st);
  return bf16 ? launch_dequant_dt<BF16, false>(p, max_bits, st) : launch_dequant_dt<F16, false>(p, max_bits, st);
}

int launch_sigma_chunks(const uint16_t* x, int64_t ldx, int M, int K, int dtype, float* partial, uint8_t* flags,
                        float* sigma, const uint16_t* scale, int64_t n_scale, uint32_t* slots, hipStream_t st) {
  if (M <= 0 || K <= 0 || K % 8 != 0) return GRINQH_ERR_INVALID;
  const int rows = sigma_chunk_rows(M), chunks = (M + rows - 1) / rows;
  const dim3 grid((unsigned)((K + 255) / 256), (unsigned)chunks);
  if (dtype == GRINQH_DTYPE_BF16)
    hipLaunchKernelGGL(sigma_chunks_kernel<BF16>, grid, dim3(256), 0, st, x, ldx, M, K, rows, partial, flags);
  else
    hipLaunchKernelGGL(sigma_chunks_kernel<F16>, grid, dim3(256), 0, st, x, ldx, M, K, rows, partial, flags);
  hipLaunchKernelGGL(sigma_chunks_reduce_kernel, dim3((unsigned)scale_range_slots(K)), dim3(256), 0, st, partial,
                     chunks, K, sigma, scale, n_scale, scale != nullptr ? slots : nullptr);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_nonfinite_rows_to_nan(const uint8_t* flags, int M, int K, uint16_t* y, int N, int dtype, hipStream_t st) {
  if (M <= 0) return GRINQH_OK;
  const uint16_t nan = dtype == GRINQH_DTYPE_BF16 ? 0x7FC0u : 0x7E00u;
  hipLaunchKernelGGL(nonfinite_rows_to_nan_kernel, dim3((unsigned)M), dim3(256), 0, st, flags, (K + 255) / 256, M, y,
                     N, nan);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_add_bias_rows(uint16_t* y, const uint16_t* bias, int64_t M, int N, int dtype, hipStream_t st) {
  if (M <= 0 || bias == nullptr) return GRINQH_OK;
  if (N % 8 != 0 || (reinterpret_cast<uintptr_t>(y) & 15u) || (reinterpret_cast<uintptr_t>(bias) & 15u))
    return GRINQH_ERR_INVALID;
  const int64_t chunks = M * (N / 8);
  const dim3 grid((unsigned)((chunks + 255) / 256));
  if (dtype == GRINQH_DTYPE_BF16)
    hipLaunchKernelGGL(add_bias_rows_kernel<BF16>, grid, dim3(256), 0, st, y, bias, M, N);
  else
    hipLaunchKernelGGL(add_bias_rows_kernel<F16>, grid, dim3(256), 0, st, y, bias, M, N);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
