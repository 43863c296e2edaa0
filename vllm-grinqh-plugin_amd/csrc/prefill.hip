// Prefill-regime GRINQH product (M > 64, below the library-GEMM path of
// dequant.hip / blas.hip): dequantize-into-LDS GEMM on
// v_mfma_f32_16x16x32_{f16,bf16}, MFMA-bound.
//
// Replaces grinqh_prefill_gemm_compiled (grinqh/kernel.py:561-587: Wd =
// RNE(W * s) in the activation dtype, then X @ Wd with fp32 accumulation) and,
// for max_bits == 4, the Marlin path (:528-558), which computes the same
// product.  The dense weight is never written to HBM: each 32-row stage of the
// B tile is rebuilt from the plane words straight into LDS as RNE(w * s),
// which is S9's rounding of the weight.
//
// Graded (union) batches use the same kernel with the per-row zone set of
// sigma_k = max_m |x[m][k]| (computed beforehand over the whole batch): the
// planes of inactive zones are masked to zero and the row's midpoint bias is
// added, i.e. the weight is RNE(w_eff * s).  The reference has no prefill
// kernel for this mode (its batch-union GEMV, grinqh/kernel.py:170-360, keeps
// fp32 products), so this path is held to the reference within the fp16
// rounding bound of the dequantized weight.
//
// Tiles: a block computes BM rows x 256 logical columns (16 plane-word columns
// x 16 column tiles) with 8 waves, two per SIMD, as (BM/64 or 4) x 2.  Per
// stage of BK rows of K: A (x) and the dequantized B go to the LDS buffer the
// MFMAs are not reading, while the global loads of the next one or two
// stages are in flight (register slots).
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

// One block: BM rows x 256 logical columns; WAVES waves as (WAVES/2) x 2, each
// BM/(WAVES/2) rows x 8 column tiles.  A stage is BK rows of K: its global
// loads are issued PD stages before its dequantization into LDS (PD register
// slots), so they are in flight while the stages before it are multiplied.
// Each dequantizing thread owns one word column, BK/16 rows and 4*JPT column
// tiles.  OCC is the occupancy hint of the launch bounds.
template <typename DT, int BM, int Z, bool DENSE, int WAVES, int BK, int OCC, int PD, bool WS = false>
__global__ __launch_bounds__(WAVES * 64, OCC) void prefill_kernel(PrefillParams p) {
  constexpr int NT = WAVES * 64;
  // WS (warp-specialised): the first half of the waves only load and
  // dequantize stages, the second half only multiply; each SIMD runs one of
  // each, so one's VALU work overlaps the other's MFMAs
  constexpr int NP = WS ? NT / 2 : NT;            // loading / dequantizing threads
  constexpr int SH = 8 - 2 * Z;
  constexpr int KP = BK + 8;        // halves per LDS row (padding: conflict-free fragment reads)
  constexpr int WGM = WS ? 2 : WAVES / 2;  // multiplying waves along M (2 along N)
  constexpr int WM = BM / WGM;      // rows per wave
  constexpr int MTW = WM / 16;      // 16-row MFMA tiles per wave
  constexpr int CPR = BK / 8;       // 16-byte x chunks per row per stage
  constexpr int AL = BM * CPR / NP;
  constexpr int RPT = BK / 16;      // rows per dequantizing thread
  constexpr int JPT = 4 * 256 / NP; // output dwords j per dequantizing thread
  static_assert(!WS || (WAVES == 8 && PD == 2), "warp-specialised shape");
  static_assert(MTW >= 1 && AL >= 1 && RPT % 2 == 0 && JPT >= 1, "tile shape");

  __shared__ __align__(16) uint16_t s_a[2][BM * KP];
  __shared__ __align__(16) uint16_t s_b[2][256 * KP];  // (column tile, column) rows of BK k

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int cw = WS ? wave - NP / 64 : wave;  // index among the multiplying waves
  const int wm = cw % WGM, wn = cw / WGM;
  const int c = lane & 15, q = lane >> 4;
  const int w0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * BM;
  // this block's K range: stages [s_begin, s_end) of BK rows
  const int nstages_all = p.K / BK;
  const int s_begin = blockIdx.z * p.stages_per_split;  // < nstages_all: no empty range is launched
  const int s_end = min(s_begin + p.stages_per_split, nstages_all);

  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.x), (short)0, (int)((uint64_t)p.M * p.ldx * 2u), 0x00020000);
  const int wcol = tid & 15, rg = (tid >> 4) & 15, j0 = (tid >> 8) * JPT;
  const bool col_ok_ld = (w0 + wcol) < p.NW;
  const int wc_ld = col_ok_ld ? (w0 + wcol) : (p.NW - 1);
  const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.planes), (short)0, (int)((uint64_t)p.K * (uint32_t)(Z * p.NW) * 4u), 0x00020000);
  const uint32_t plane_row_bytes = (uint32_t)(Z * p.NW) * 4u;
  // scales through a buffer descriptor: the group's row offset is one scalar,
  // this thread's column offset one register (no 64-bit address per scale)
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.scale), (short)0, (int)((uint64_t)((p.K + p.gs - 1) / p.gs) * p.N * 2u), 0x00020000);
  const uint32_t s_col_off = ((uint32_t)(4 * j0) * (uint32_t)p.NW + (uint32_t)wc_ld) * 2u;

  // Graded fp16: RNE(w * s) overflows where |w| * |s| > 65504 (|w| <= 2^(2Z-1)),
  // which the fp32 products of the reference's union GEMV do not.  A block
  // whose scales (its K range, its 256 columns) reach past kScaleLimit builds
  // B from s * 2^-e and scales its sums by 2^e (both exact, except for scales
  // that become subnormal).  Read once before the main loop.
  constexpr bool GUARD = !DENSE && DT::id == F16::id;
  constexpr uint32_t kScaleLimit = 0x7BFFu - ((uint32_t)(2 * Z - 1) << 10);  // 65504 / 2^(2Z-1), fp16 bits
  int up_exp = 0;
  if constexpr (GUARD) {
    __shared__ uint32_t s_wmax[WAVES];
    const int g_lo = (s_begin * BK) / p.gs, g_hi = (s_end * BK - 1) / p.gs;
    const int total = (g_hi - g_lo + 1) * 256;  // (group, column tile, word column)
    uint32_t hm = 0;
    for (int i0 = tid; i0 < total; i0 += NT * 8) {
      uint16_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = i0 + NT * u;
        const int col = ((idx >> 4) & 15) * p.NW + min(w0 + (idx & 15), p.NW - 1);
        const uint32_t off = idx < total ? ((uint32_t)(g_lo + (idx >> 8)) * (uint32_t)p.N + (uint32_t)col) * 2u
                                         : 0x80000000u;
        v[u] = __builtin_amdgcn_raw_buffer_load_b16(srsrc, (int)off, 0, 0);
      }
#pragma unroll
      for (int u = 0; u < 8; ++u) hm = max(hm, (uint32_t)v[u] & 0x7FFFu);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) hm = max(hm, (uint32_t)__shfl_xor((int)hm, o, 64));
    if (lane == 0) s_wmax[wave] = hm;
    __syncthreads();
#pragma unroll
    for (int w = 0; w < WAVES; ++w) hm = max(hm, s_wmax[w]);
    if (hm > kScaleLimit) up_exp = (int)(hm >> 10) - (int)(kScaleLimit >> 10);
  }
  const float down_scale = __builtin_ldexpf(1.f, -up_exp), up_scale = __builtin_ldexpf(1.f, up_exp);

  // registers of one stage's global loads; PD stages are in flight at once
  struct Slot {
    u32x4_t xa[AL];
    uint32_t D[RPT][Z];
    float sig[RPT];
    uint16_t sraw[4 * JPT];  // scales of the stage's group when it starts a new group
    bool new_group;
  };
  auto load_stage = [&](int s, Slot& L) {
    const int k0 = s * BK;
    L.new_group = (s == s_begin) || (k0 / p.gs != (k0 - BK) / p.gs);
    if (L.new_group) {  // this thread's columns: column tiles 4*j0 .., word column wc_ld
      const int g = k0 / p.gs;
#pragma unroll
      for (int r = 0; r < 4 * JPT; ++r)
        L.sraw[r] = __builtin_amdgcn_raw_buffer_load_b16(srsrc, (int)(s_col_off + (uint32_t)r * (uint32_t)p.NW * 2u),
                                                       (int)((uint32_t)g * (uint32_t)p.N * 2u), 0);
    }
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const int h = tid + NP * i, row = h / CPR, piece = h % CPR;
      const int m = m0 + row;
      const uint32_t off = m < p.M ? (uint32_t)(((int64_t)m * p.ldx + k0 + 8 * piece) * 2) : 0x80000000u;
      L.xa[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
    }
    // every plane of the stage's rows; graded batches mask the inactive ones
    // when the stage is stored (fetching only the active ones measured slower)
#pragma unroll
    for (int e = 0; e < RPT; ++e) {
      const int row = k0 + rg * RPT + e;
      const uint32_t rb = (uint32_t)row * plane_row_bytes + (uint32_t)wc_ld * 4u;
#pragma unroll
      for (int z = 0; z < Z; ++z)
        L.D[e][z] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(prsrc, (int)(rb + (uint32_t)z * p.NW * 4u), 0, 0);
      if constexpr (!DENSE) L.sig[e] = p.sigma[row];
    }
  };

  uint32_t s2[4 * JPT];  // fp16: (s, s)
  float sf[4 * JPT];     // bf16: s * 2^-sh

  // x rows as they are; B: grade (union), rebuild code bytes, RNE(w * s),
  // written as (column tile, column)[k]
  auto store_stage = [&](int buf, Slot& L) {
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const int h = tid + NP * i, row = h / CPR, piece = h % CPR;
      *reinterpret_cast<u32x4_t*>(&s_a[buf][row * KP + 8 * piece]) = L.xa[i];
    }
    int beta[RPT];
#pragma unroll
    for (int e = 0; e < RPT; ++e) {
      const uint32_t bits = DENSE ? ((1u << Z) - 1u) : zone_bits<Z>(L.sig[e], p.thr.t);
      beta[e] = DENSE ? 0 : midpoint_bias<Z>(bits);
      if (!DENSE) {
#pragma unroll
        for (int z = 0; z < Z; ++z) L.D[e][z] &= 0u - ((bits >> z) & 1u);
      }
      L.D[e][0] ^= 0xAAAAAAAAu;  // offset binary: u = int8(U & mask) + 128
#pragma unroll
      for (int z = 1; z < Z; ++z) L.D[e][z] = rotr(L.D[e][z], (uint32_t)(2 * z));
    }
    if (L.new_group) {
#pragma unroll
      for (int r = 0; r < 4 * JPT; ++r) {
        if constexpr (DT::id == F16::id) {
          const uint16_t sh = (GUARD && up_exp > 0) ? from_f32<DT>(to_f32<DT>(L.sraw[r]) * down_scale) : L.sraw[r];
          s2[r] = (uint32_t)sh | ((uint32_t)sh << 16);
        }
        else
          sf[r] = to_f32<DT>(L.sraw[r]) * (1.0f / (float)(1 << SH));
      }
    }
#pragma unroll
    for (int pp = 0; pp < RPT / 2; ++pp) {
      uint32_t negc = 0;
      float cb0 = 0.f, cb1 = 0.f;
      if constexpr (DT::id == F16::id) {
        const uint16_t c0 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[2 * pp]));
        const uint16_t c1 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[2 * pp + 1]));
        negc = (uint32_t)c0 | ((uint32_t)c1 << 16);
      } else {
        cb0 = (float)(128 - beta[2 * pp] * (1 << SH));
        cb1 = (float)(128 - beta[2 * pp + 1] * (1 << SH));
      }
      uint16_t* bdst = &s_b[buf][wcol * KP + rg * RPT + 2 * pp];
#pragma unroll
      for (int jj = 0; jj < JPT; ++jj) {
        const int j = j0 + jj;
        uint32_t V[2];
#pragma unroll
        for (int e = 0; e < 2; ++e) {
          const int ee = 2 * pp + e;
          uint32_t h = (Z == 4) ? L.D[ee][3] : (L.D[ee][0] & (0x03030303u << (2 * ((3 - j) & 3))));
#pragma unroll
          for (int z = (Z == 4 ? 0 : 1); z < (Z == 4 ? 3 : Z); ++z)
            h = bfi(0x03030303u << (2 * ((3 - z - j) & 3)), L.D[ee][z], h);
          V[e] = rotr(h, (uint32_t)(32 - 2 * j) & 31u);
        }
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const int r = 4 * j + b;
          uint32_t pr;
          if constexpr (DT::id == F16::id) {
            pr = Dequant<F16, SH>::pair(V[0], V[1], b, negc, s2[4 * jj + b]);
          } else {
            pr = Dequant<BF16, SH>::pair_bf16(V[0], V[1], b, cb0, cb1, sf[4 * jj + b]);
          }
          *reinterpret_cast<uint32_t*>(bdst + r * 16 * KP) = pr;
        }
      }
    }
  };

  f32x4_t acc[MTW][8];
#pragma unroll
  for (int i = 0; i < MTW; ++i)
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[i][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // MFMAs of one stage from LDS buffer buf.  All fragments of a 32-deep k step
  // are read before its MFMAs, and the next k step's fragments are read while
  // they run, so the matrix core is not left waiting on LDS between tiles.
  auto multiply_stage = [&](int buf) {
    u32x4_t Bf[2][8], Af[2][MTW];
    auto read_frags = [&](int ks, int f) {
#pragma unroll
      for (int r = 0; r < 8; ++r)
        Bf[f][r] = *reinterpret_cast<const u32x4_t*>(&s_b[buf][((8 * wn + r) * 16 + c) * KP + 32 * ks + 8 * q]);
#pragma unroll
      for (int i = 0; i < MTW; ++i)
        Af[f][i] = *reinterpret_cast<const u32x4_t*>(&s_a[buf][(wm * WM + 16 * i + c) * KP + 32 * ks + 8 * q]);
    };
    read_frags(0, 0);
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      if (ks + 1 < BK / 32) read_frags(ks + 1, (ks + 1) & 1);
      __builtin_amdgcn_sched_barrier(0);  // keep the reads ahead of the MFMAs
#pragma unroll
      for (int i = 0; i < MTW; ++i)
#pragma unroll
        for (int r = 0; r < 8; ++r) acc[i][r] = mfma16x16x32<DT>(Af[ks & 1][i], Bf[ks & 1][r], acc[i][r]);
    }
  };

  // The loop bodies below load and store unconditionally: with the loads
  // always consumed inside the body the compiler's wait counts stay exact (a
  // conditional store made it wait for every outstanding load, scale loads
  // included, at the top of each stage).  Stage t is multiplied from LDS
  // buffer (t - s_begin) & 1.
  Slot LA, LB;
  int s = s_begin;
  if constexpr (WS) {
    // Both roles pass the same number of barriers: one after the first
    // stage is stored, then one per stage but the last.  Stage t lives in
    // LDS buffer (t - s_begin) & 1 and in register slot (t - s_begin) & 1
    // (LA even, LB odd); two stages of loads are in flight.  Loads past the
    // range repeat its last stage (unconditional loads keep the wait counts
    // exact) and are never stored.
    if (wave < NP / 64) {
      const int last = s_end - 1;
      load_stage(s_begin, LA);
      store_stage(0, LA);
      load_stage(min(s_begin + 1, last), LB);
      load_stage(min(s_begin + 2, last), LA);
      __syncthreads();
      for (; s + 2 < s_end; s += 2) {  // store stages s+1 and s+2
        store_stage(1, LB);
        load_stage(min(s + 3, last), LB);
        __syncthreads();
        store_stage(0, LA);
        load_stage(min(s + 4, last), LA);
        __syncthreads();
      }
      if (s + 1 < s_end) {  // store stage s+1
        store_stage(1, LB);
        __syncthreads();
      }
      return;  // the multiplying waves write the output
    }
    __syncthreads();
    for (; s + 1 < s_end; ++s) {
      multiply_stage((s - s_begin) & 1);
      __syncthreads();
    }
    multiply_stage((s - s_begin) & 1);
  } else if constexpr (PD == 1) {
    load_stage(s_begin, LA);
    store_stage(0, LA);
    __syncthreads();
    for (; s + 1 < s_end; ++s) {  // stage s+1 loads while stage s is multiplied
      const int buf = (s - s_begin) & 1;
      load_stage(s + 1, LA);
      multiply_stage(buf);
      store_stage(buf ^ 1, LA);
      __syncthreads();
    }
    multiply_stage((s - s_begin) & 1);
  } else {
    // two stages in flight: at the top of each iteration stage s is in LDS
    // buffer 0 and stage s+1 is loading into LB (a single-stage range loads
    // its stage twice, harmlessly)
    load_stage(s_begin, LA);
    store_stage(0, LA);
    load_stage(s + 1 < s_end ? s + 1 : s, LB);
    __syncthreads();
    for (; s + 3 < s_end; s += 2) {
      load_stage(s + 2, LA);
      multiply_stage(0);
      store_stage(1, LB);
      __syncthreads();
      load_stage(s + 3, LB);
      multiply_stage(1);
      store_stage(0, LA);
      __syncthreads();
    }
    if (s + 2 < s_end) {  // stages s, s+1, s+2 left
      load_stage(s + 2, LA);
      multiply_stage(0);
      store_stage(1, LB);
      __syncthreads();
      multiply_stage(1);
      store_stage(0, LA);
      __syncthreads();
      multiply_stage(0);
    } else if (s + 1 < s_end) {  // stages s, s+1 left
      multiply_stage(0);
      store_stage(1, LB);
      __syncthreads();
      multiply_stage(1);
    } else {
      multiply_stage(0);
    }
  }

  // epilogue: lane (c, q) holds rows 4q..4q+3 of each 16 x 16 tile
  const bool col_ok = (w0 + c) < p.NW;
  if (!col_ok) return;
#pragma unroll
  for (int i = 0; i < MTW; ++i)
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const int64_t n = (int64_t)(8 * wn + r) * p.NW + w0 + c;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = m0 + wm * WM + 16 * i + 4 * q + e;
        if (m >= p.M) continue;
        const float v = DENSE ? acc[i][r][e] : graded_nonfinite_to_nan(GUARD ? acc[i][r][e] * up_scale : acc[i][r][e]);
        if (p.splits == 1)
          p.y[(int64_t)m * p.N + n] = finish_output<DT>(v, p.bias, (int)n);
        else
          p.partial[((int64_t)blockIdx.z * p.M + m) * p.N + n] = v;
      }
    }
}

template <typename DT, int BM, int Z, int WAVES, int BK, int PD, bool WS>
static void launch_prefill_t(const PrefillParams& p0, bool dense, hipStream_t st) {
  PrefillParams p = p0;  // K ranges of whole BK stages, none empty
  const int nst = p.K / BK;
  p.stages_per_split = (nst + p0.splits - 1) / p0.splits;
  p.splits = (nst + p.stages_per_split - 1) / p.stages_per_split;
  const dim3 grid((p.NW + 15) / 16, (p.M + BM - 1) / BM, p.splits);
  if (dense)
    launch_main_kernel(prefill_kernel<DT, BM, Z, true, WAVES, BK, 1, PD, WS>, grid, dim3(WAVES * 64), st, p);
  else
    launch_main_kernel(prefill_kernel<DT, BM, Z, false, WAVES, BK, 1, PD, WS>, grid, dim3(WAVES * 64), st, p);
}

template <typename DT, int BM, int WAVES, int BK, int PD, bool WS = false>
static int launch_prefill_bm(const PrefillParams& p, int Z, bool dense, hipStream_t st) {
  switch (Z) {
    case 1: launch_prefill_t<DT, BM, 1, WAVES, BK, PD, WS>(p, dense, st); break;
    case 2: launch_prefill_t<DT, BM, 2, WAVES, BK, PD, WS>(p, dense, st); break;
    case 3: launch_prefill_t<DT, BM, 3, WAVES, BK, PD, WS>(p, dense, st); break;
    case 4: launch_prefill_t<DT, BM, 4, WAVES, BK, PD, WS>(p, dense, st); break;
    default: return GRINQH_ERR_INVALID;
  }
  return GRINQH_OK;
}

// 256-row tiles when they still give one block per CU, else 128-row tiles.
int prefill_block_rows(int64_t M, int64_t N) {
  const int64_t col_blocks = (N / 16 + 15) / 16;
  return col_blocks * ((M + 255) / 256) >= kTargetBlocks ? 256 : 128;
}

int prefill_splits(int64_t M, int64_t K, int64_t N) {
  const int64_t BM = prefill_block_rows(M, N);
  const int64_t blocks = ((N / 16 + 15) / 16) * ((M + BM - 1) / BM);
  int64_t cap = (kTargetBlocks + blocks - 1) / blocks;  // enough ranges for a block per CU
  const int64_t by_k = K / 256;
  if (cap > by_k) cap = by_k;
  const int64_t by_bytes = (int64_t)kMaxPrefillPartialBytes / (M * N * 4);
  if (cap > by_bytes) cap = by_bytes;
  // One block per CU: a launch takes ceil(blocks * s / 256) rounds of K / s
  // rows each.  Take the s <= cap with the fewest rounds per range (the
  // fewest ranges on a tie): 24 column blocks split 11 ways would start a
  // second round for 8 blocks, split 10 ways they fit one.
  int64_t best = 1;
  for (int64_t s = 2; s <= cap; ++s) {
    const int64_t rounds = (blocks * s + kTargetBlocks - 1) / kTargetBlocks;
    const int64_t best_rounds = (blocks * best + kTargetBlocks - 1) / kTargetBlocks;
    if (rounds * best < best_rounds * s) best = s;
  }
  return (int)best;
}

// Stage rows and stages in flight per configuration.  256-row tiles (fp16,
// grid of at least one block per CU): 8 waves, two per SIMD (64 x 128 per
// wave), 32-row stages, one stage in flight (64-row stages or a second stage
// do not fit 256 registers).  128-row tiles: fp16 dense batches run the
// warp-specialised form (4 waves load and dequantize 32-row stages with two
// stages in flight, 4 waves of 64 x 128 multiply), dense or graded; bf16
// runs 8 waves of 32 x 128 with 64-row stages (when K and the group size
// allow) and one stage in flight.  Two waves per SIMD let one wave's
// dequantization and loads overlap the other's MFMAs.
struct PrefillShape {
  int bm, bk, pd;
};
static PrefillShape prefill_shape(const PrefillParams& p, int dtype) {
  const bool bk64 = (p.K % 64 == 0) && (p.gs % 64 == 0);
  // (bf16's fp32 dequantization does not fit the 256-row tile's registers:
  // it always takes 128-row tiles)
  if (dtype == GRINQH_DTYPE_F16 && prefill_block_rows(p.M, p.N) == 256) return {256, 32, 1};
  if (dtype == GRINQH_DTYPE_F16) return {128, 32, 2};
  return {128, bk64 ? 64 : 32, 1};
}

template <typename DT>
static int launch_prefill_dt(const PrefillParams& p, const PrefillShape& sh, int Z, bool dense, hipStream_t st) {
  if constexpr (DT::id == F16::id) {  // the shapes only fp16 takes
    if (sh.bm == 256) return launch_prefill_bm<DT, 256, 8, 32, 1>(p, Z, dense, st);
    if (sh.pd == 2) return launch_prefill_bm<DT, 128, 8, 32, 2, true>(p, Z, dense, st);
  }
  return sh.bk == 64 ? launch_prefill_bm<DT, 128, 8, 64, 1>(p, Z, dense, st)
                     : launch_prefill_bm<DT, 128, 8, 32, 1>(p, Z, dense, st);
}

// K ranges launch_prefill_t runs for an upper bound `splits` (whole stages).
static int prefill_splits_run(const PrefillParams& p, int splits, int bk) {
  const int nst = p.K / bk;
  const int sps = (nst + splits - 1) / splits;
  return (nst + sps - 1) / sps;
}

int launch_prefill(const PrefillParams& p, int max_bits, int dtype, bool dense, hipStream_t st,
                   int* splits_run) {
  if (!dense && p.sigma == nullptr) return GRINQH_ERR_INVALID;
  if (p.splits < 1 || (p.splits > 1 && p.partial == nullptr)) return GRINQH_ERR_INVALID;
  const PrefillShape sh = prefill_shape(p, dtype);
  *splits_run = prefill_splits_run(p, p.splits, sh.bk);
  const int Z = max_bits / 2;
  const int rc = dtype == GRINQH_DTYPE_BF16 ? launch_prefill_dt<BF16>(p, sh, Z, dense, st)
                                            : launch_prefill_dt<F16>(p, sh, Z, dense, st);
  if (rc != GRINQH_OK) return rc;
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
