// GEMV-regime GRINQH product (M <= 4 per launch): graded or dense
// y = x * W_eff on v_mfma_f32_16x16x32_{f16,bf16}, HBM-bound.
//
// Replaces the reference's Triton GEMV grinqh_gemv_uint32_packed
// (grinqh/kernel.py:39-167, one row), the batch-union GEMV
// grinqh_gemv_uint32_packed_batch_union (:170-360) for batches of up to four
// rows, and the dense branch of grinqh_gemm_or_gemv for such batches
// (:663-680, semantics of :561-587).
//
// Each lane owns one plane-word column w = w0 + lane (16 logical columns,
// one per column tile 4j+beta), so every buffer load of a wave reads one
// 256-byte run of a (row, plane) line, and a (row, plane) the grading skips is
// skipped by the whole wave.  The MFMA is used block-diagonally: lane (c, q)
// supplies B = the 8 rows of the tile for its own column w, and A holds x
// rows 0..3 only in the q-th 4x8 block of the 16x32 A tile:
//   A[m][8q' + e] = x[m & 3][row e]  if m >> 2 == q'  else 0,
// so output rows 4q..4q+3 of column c are y[0..3] of word column 16q + c,
// exactly the lane that holds them.
//
// Work decomposition
//   grid.x = 64 word columns (1024 logical columns), grid.y = K range; two
//   blocks per CU
//   4 waves = 4 consecutive sub-ranges of the K range (8-row tiles for one
//   row, 4-row tiles on v_mfma_f32_16x16x16 for two to four), reduced through
//   LDS in fixed order; the K ranges of the grid are added by the range that
//   finishes last (small reductions) or by the split-K reduction kernel.
#include "grinqh_common.h"
#include "grinqh_launch.h"
#include "splitk_complete.h"

namespace grinqh {

constexpr int kGemvRowsPerBlock = 1024;   // rows of x staged per block
constexpr int kGemvScaleGroups = 9;       // scale groups staged per block
// Two resident blocks per CU (256 registers per lane) for one row on 8-row
// tiles and for up to four rows on 4-row tiles.
constexpr int gemv_tile_rows(int mr) { return mr == 1 ? 8 : 4; }
constexpr int gemv_blocks_per_cu(int) { return 2; }

// Tiles of TR rows: 8 rows on v_mfma_f32_16x16x32 (one x row), 4 rows on
// v_mfma_f32_16x16x16 (up to four x rows: half the plane words in flight per
// tile, which leaves room for the 64 accumulators at two blocks per CU).
template <int TR>
struct GemvTile;
template <>
struct GemvTile<8> {
  typedef u32x4_t vec_t;
};
template <>
struct GemvTile<4> {
  typedef u32x2_t vec_t;
};
template <typename DT, int TR>
__device__ __forceinline__ f32x4_t tile_mfma(const typename GemvTile<TR>::vec_t& a,
                                             const typename GemvTile<TR>::vec_t& b, f32x4_t c) {
  if constexpr (TR == 8)
    return mfma16x16x32<DT>(a, b, c);
  else
    return mfma16x16x16<DT>(a, b, c);
}

template <typename DT, int MR, int Z, bool DENSE>
__global__ __launch_bounds__(256, gemv_blocks_per_cu(MR)) void gemv_kernel(DecodeParams p) {
  constexpr int SH = 8 - 2 * Z;
  constexpr int TR = gemv_tile_rows(MR);
  constexpr int RMAX = kGemvRowsPerBlock;
  constexpr int XS = RMAX + 8;                 // halves per staged x row
  constexpr int X_BYTES = 5 * XS * 2;          // x rows 0..3, row 4 all zero
  constexpr int OFF_BYTES = RMAX * Z * 4;
  constexpr int RED_BYTES = 3 * 16 * MR * 64 * 4;  // each dword's sums of the three waves not owning it
  constexpr int POOL_BYTES = (X_BYTES + OFF_BYTES) > RED_BYTES ? (X_BYTES + OFF_BYTES) : RED_BYTES;
  constexpr int SCG = kGemvScaleGroups;
  constexpr int CPR = RMAX / 8;                // 16-byte chunks per staged x row
  constexpr int XPT = 4 * CPR / 256;
  constexpr int SCH = SCG * 16 * 8;            // 16-byte scale chunks (group, tile, 8 columns)
  constexpr int SPT = (SCH + 255) / 256;

  __shared__ __align__(16) unsigned char s_pool[POOL_BYTES];
  __shared__ __align__(16) uint16_t s_bv[RMAX];               // row -> correction-column value
  __shared__ __align__(16) uint32_t s_xm[RMAX];               // row -> zone-0 flip
  __shared__ __align__(16) uint16_t s_scale[SCG * 16 * 64];   // (group, tile, word column) scales
  uint16_t* s_x = reinterpret_cast<uint16_t*>(s_pool);
  uint32_t* s_off = reinterpret_cast<uint32_t*>(s_pool + X_BYTES);
  float* s_red = reinterpret_cast<float*>(s_pool);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int w0 = blockIdx.x * 64;
  const int split = blockIdx.y;
  const int tile0 = split * p.tiles_per_split;
  const int tile1 = min(tile0 + p.tiles_per_split, p.K >> 5);
  const int R = (tile1 - tile0) * 32;
  const int row0 = tile0 * 32;
  const int g_first = row0 / p.gs;
  const int n_groups = (row0 + R - 1) / p.gs - g_first + 1;
  // lanes past the last word column read the last valid one (never stored)
  const bool col_ok = (w0 + lane) < p.NW;
  const int wc = col_ok ? (w0 + lane) : (p.NW - 1);

  // ---- phase 1a: stage x rows 0..3 of [row0, row0 + R); the scales are loaded
  // here and stored to LDS only once the first tiles' plane loads are issued
  // (they are needed at the first group's end), so their memory round trip
  // overlaps those loads.  Out-of-range offsets read 0: rows m >= M stage as zeros.
  const bool vec_scales = (p.NW % 8) == 0 && (reinterpret_cast<uintptr_t>(p.scale) & 15u) == 0;
  u32x4_t sv[SPT];
  {
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.x), (short)0, (int)((uint64_t)p.M * p.ldx * 2u), 0x00020000);
    const uint32_t sbytes = (uint32_t)((uint64_t)((p.K + p.gs - 1) / p.gs) * p.N * 2u);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.scale), (short)0, (int)sbytes, 0x00020000);
    u32x4_t xv[XPT];
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int h = tid + 256 * k, m = h / CPR, u = h % CPR;
      const uint32_t off =
          (m < p.M && 8 * u < R) ? (uint32_t)(((int64_t)m * p.ldx + row0 + 8 * u) * 2) : 0x80000000u;
      xv[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
    }
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int h = tid + 256 * k;
      const int gl = h >> 7, r = (h >> 3) & 15, h8 = h & 7;
      const uint32_t off =
          (h < SCH && gl < n_groups && vec_scales)
              ? (uint32_t)(((int64_t)(g_first + gl) * p.N + (int64_t)r * p.NW + w0 + 8 * h8) * 2)
              : 0x80000000u;
      sv[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(sr, (int)off, 0, 0));
    }
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      const int h = tid + 256 * k, m = h / CPR, u = h % CPR;
      *reinterpret_cast<u32x4_t*>(&s_x[m * XS + 8 * u]) = xv[k];
    }
    if (tid < CPR) *reinterpret_cast<u32x4_t*>(&s_x[4 * XS + 8 * tid]) = u32x4_t{0u, 0u, 0u, 0u};
  }
  __syncthreads();

  // ---- phase 1b: grade each row: correction-column value, zone-0 flip and plane
  // offsets (w_eff * 2^sh = u + beta * 2^sh - (zone 0 active ? 128 : 0), with u the
  // offset-binary byte when zone 0 is active, else U & mask).  The statistic
  // comes from the staged x, or from the caller (a batch split into several
  // launches, a producer's chunk maxima); the two loops are separate so that
  // the first has no global load, and the scale loads stay in flight through it.
  auto grade_row = [&](int rr, float s) {
    uint32_t bits = (1u << Z) - 1u;
    if constexpr (!DENSE) bits = zone_bits<Z>(s, p.thr.t);
    const int beta = DENSE ? 0 : midpoint_bias<Z>(bits);
    s_bv[rr] = BOperand<DT>::correction(beta * (1 << SH) - ((bits & 1u) ? 128 : 0));
    s_xm[rr] = zone0_flip(bits);
    const uint32_t row_bytes = (uint32_t)(row0 + rr) * (uint32_t)(Z * p.NW) * 4u;
#pragma unroll
    for (int z = 0; z < Z; ++z)
      s_off[rr * Z + z] = ((bits >> z) & 1u) ? row_bytes + (uint32_t)z * (uint32_t)p.NW * 4u : 0x80000000u;
  };
  if (DENSE || p.sigma == nullptr) {
    for (int rr = tid; rr < R; rr += 256) {
      float s = 0.f;
      if constexpr (!DENSE) {
        s = fabsf(to_f32<DT>(s_x[rr]));
        for (int m = 1; m < p.M; ++m) s = fmaxf(s, fabsf(to_f32<DT>(s_x[m * XS + rr])));
      }
      grade_row(rr, s);
    }
  } else {
    for (int rr = tid; rr < R; rr += 256) grade_row(rr, precomputed_sigma(p, row0 + rr));
  }
  __syncthreads();

  // ---- phase 2: this wave's TR-row tiles
  typedef typename GemvTile<TR>::vec_t vec_t;
  f32x4_t C[4][4];
  f32x4_t Cv;
  float Y[4][4][MR];
#pragma unroll
  for (int j = 0; j < 4; ++j)
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int i = 0; i < MR; ++i) Y[j][b][i] = 0.f;

  const float post = BOperand<DT>::kUnit / (float)(1 << SH);
  const int nt = R / TR;
  const int t_begin = (nt * wave) >> 2, t_end = (nt * (wave + 1)) >> 2;
  // A operand rows: lane (c, q) carries x row c & 3 when c >> 2 == q, else the zero row
  const uint16_t* a_row = s_x + (((c >> 2) == q) ? (c & 3) : 4) * XS;

  // Raw buffer loads; a (row, plane) the grading skips has offset bit 31 set
  // (past the end: reads 0, no memory access).  Tiles past the end of the
  // wave's range use a descriptor of size 0.  Every load is issued, so wait
  // counts are static with two tiles in flight.
  const int plane_bytes = (int)((uint64_t)p.K * (uint32_t)(Z * p.NW) * 4u);
  const __amdgpu_buffer_rsrc_t prsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p.planes), (short)0, plane_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t prsrc_none =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p.planes), (short)0, 0, 0x00020000);
  const uint32_t lane_off = (uint32_t)wc * 4u;

  typedef uint32_t offz_t __attribute__((ext_vector_type(Z)));
  auto issue = [&](int t, uint32_t (&D)[TR][Z]) {
    const bool live = t < t_end;
    const __amdgpu_buffer_rsrc_t rs = live ? prsrc : prsrc_none;
    const int sb = (live ? t : t_begin) * TR;
#pragma unroll
    for (int e = 0; e < TR; ++e) {
      offz_t o;
      if constexpr (Z == 1) {
        o = s_off[sb + e];
      } else {
        o = *reinterpret_cast<const offz_t*>(&s_off[(sb + e) * Z]);
      }
#pragma unroll
      for (int z = 0; z < Z; ++z) {
        const uint32_t oz = (Z == 1) ? (uint32_t)o[0] : (uint32_t)o[z];
        D[e][z] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)(oz + lane_off), 0, 0);
      }
    }
  };

  // position of the current tile in its scale group and the group's index in
  // the staged scales, advanced per tile (no divisions in the loop)
  const int tiles_per_group = p.gs / TR;
  int gpos = (row0 / TR + t_begin) % tiles_per_group;
  int gloc = (row0 + TR * t_begin) / p.gs - g_first;
  auto step = [&](int t, uint32_t (&Dc)[TR][Z], bool prefetch, uint32_t (&Dn)[TR][Z]) {
    const bool first_of_group = (t == t_begin) || (gpos == 0);
    const bool last_of_group = (t + 1 == t_end) || (gpos + 1 == tiles_per_group);
    if (prefetch) issue(t + 2, Dn);
    __builtin_amdgcn_sched_barrier(0);

    const vec_t A = *reinterpret_cast<const vec_t*>(a_row + TR * t);
    const vec_t bv = *reinterpret_cast<const vec_t*>(&s_bv[TR * t]);
    uint32_t xm[TR];
#pragma unroll
    for (int h = 0; h < TR / 4; ++h) {
      const u32x4_t v = *reinterpret_cast<const u32x4_t*>(&s_xm[TR * t + 4 * h]);
#pragma unroll
      for (int e = 0; e < 4; ++e) xm[4 * h + e] = v[e];
    }
    prepare_planes<Z, TR>(Dc, xm);
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t V[TR];
      code_dwords<Z, TR>(Dc, j, V);
      vec_t B[4];
#pragma unroll
      for (int pr = 0; pr < TR / 2; ++pr)
#pragma unroll
        for (int b = 0; b < 4; ++b) B[b][pr] = BOperand<DT>::pair(V[2 * pr], V[2 * pr + 1], b);
      if (first_of_group) {
#pragma unroll
        for (int b = 0; b < 4; ++b) C[j][b] = tile_mfma<DT, TR>(A, B[b], f32x4_t{0.f, 0.f, 0.f, 0.f});
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b) C[j][b] = tile_mfma<DT, TR>(A, B[b], C[j][b]);
      }
    }
    Cv = tile_mfma<DT, TR>(A, bv, first_of_group ? f32x4_t{0.f, 0.f, 0.f, 0.f} : Cv);

    if (last_of_group) {  // y += s[g][n] * 2^-sh * (C + Cv)
      const uint16_t* srow = &s_scale[gloc * 1024 + lane];
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float sc = to_f32<DT>(srow[(4 * j + b) * 64]) * post;
#pragma unroll
          for (int i = 0; i < MR; ++i) Y[j][b][i] = fmaf(sc, C[j][b][i] + Cv[i], Y[j][b][i]);
        }
    }
    if (gpos + 1 == tiles_per_group) {
      gpos = 0;
      ++gloc;
    } else {
      ++gpos;
    }
  };

  {
    uint32_t DA[TR][Z], DB[TR][Z], DC[TR][Z];
    issue(t_begin, DA);
    issue(t_begin + 1, DB);
    // the scales, now that the first tiles' loads are in flight; the barrier
    // does not wait for those loads (no memory fence), only for the LDS stores
    // one of two staging paths per block: the 16-byte loads' zero fill (when
    // they were not issued) would race with element-wise stores to the same words
    if (vec_scales) {
#pragma unroll
      for (int k = 0; k < SPT; ++k) {
        const int h = tid + 256 * k;
        if (h < SCH) *reinterpret_cast<u32x4_t*>(&s_scale[h * 8]) = sv[k];
      }
    } else {  // element-wise staging
      for (int idx = tid; idx < n_groups * 1024; idx += 256) {
        const int gl = idx >> 10, r = (idx >> 6) & 15;
        const int wcol = min(w0 + (idx & 63), p.NW - 1);
        s_scale[idx] = p.scale[(int64_t)(g_first + gl) * p.N + (int64_t)r * p.NW + wcol];
      }
    }
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    int t = t_begin;
    for (; t + 3 <= t_end; t += 3) {
      step(t, DA, true, DC);
      step(t + 1, DB, true, DA);
      step(t + 2, DC, true, DB);
    }
    if (t < t_end) step(t, DA, false, DC);
    if (t + 1 < t_end) step(t + 1, DB, false, DC);
  }

  // ---- phase 3: add the waves' sub-ranges in order 0, 1, 2, 3.  Wave j owns
  // output dword j (columns (4j + b) * NW + w): it adds that dword's sums of
  // all four waves and writes its outputs, so that the block's stores are
  // spread over its waves (at four rows 16 per lane each, instead of 64 for
  // wave 0).  Slot (j, k') holds the sums of the k'-th other wave.
  __syncthreads();
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (wave == j) continue;
    const int k1 = wave < j ? wave : wave - 1;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int i = 0; i < MR; ++i) s_red[(((j * 3 + k1) * 4 + b) * MR + i) * 64 + lane] = Y[j][b][i];
  }
  __syncthreads();
  float O[4][MR];  // this wave's dword: the block's sums
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (wave != j) continue;
#pragma unroll
    for (int b = 0; b < 4; ++b)
#pragma unroll
      for (int i = 0; i < MR; ++i) {
        auto part = [&](int k) -> float {  // wave k's sum
          if (k == j) return Y[j][b][i];
          return s_red[(((j * 3 + (k < j ? k : k - 1)) * 4 + b) * MR + i) * 64 + lane];
        };
        float acc = part(0);
#pragma unroll
        for (int k = 1; k < 4; ++k) acc += part(k);
        O[b][i] = acc;
      }
  }

  // ---- phase 4: output column n = (4 * wave + b) * NW + w of rows m < M
  if (p.splits == 1) {
    if (col_ok) {
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int64_t n = (int64_t)(4 * wave + b) * p.NW + wc;
#pragma unroll
        for (int i = 0; i < MR; ++i)
          if (i < p.M) p.y[(int64_t)i * p.N + n] = finish_output<DT>(O[b][i], p.bias, (int)n);
      }
    }
  } else if ((int64_t)p.M * p.N * 4 < ((int64_t)1 << 31)) {
    // agent-scope (sc1) raw buffer stores without branches: rows m >= M and
    // lanes past the last word column get an offset past the K range's slab
    // (dropped by the range check); the column tile's part is the scalar offset
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(p.partial + (int64_t)split * p.M * p.N, (short)0,
                                          (int)((uint32_t)p.M * (uint32_t)p.N * 4u), 0x00020000);
    uint32_t roff[MR];
#pragma unroll
    for (int i = 0; i < MR; ++i)
      roff[i] = (i < p.M && col_ok) ? ((uint32_t)i * (uint32_t)p.N + (uint32_t)wc) * 4u : 0x80000000u;
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t coff = (uint32_t)(4 * wave + b) * (uint32_t)p.NW * 4u;  // wave-uniform
#pragma unroll
      for (int i = 0; i < MR; ++i)
        __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(O[b][i]), prs, (int)roff[i], (int)coff, kCpolSc1);
    }
  } else if (col_ok) {
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const int64_t n = (int64_t)(4 * wave + b) * p.NW + wc;
#pragma unroll
      for (int i = 0; i < MR; ++i)
        if (i < p.M) store_partial(&p.partial[((int64_t)split * p.M + i) * p.N + n], O[b][i]);
    }
  }
  // the K range that finishes last adds all ranges' partial sums of this column block
  if (p.splits > 1 && p.counters != nullptr) splitk_complete<DT, MR>(p, blockIdx.x, w0, 64);
}

// The plan sizes K ranges for a group size of 32 (the largest split count);
// larger groups give at most as many ranges, so the workspace bound holds.
DecodePlan plan_gemv(int64_t M, int64_t K, int64_t N, int64_t group_size) {
  DecodePlan pl{};
  pl.mt = 1;
  const int64_t NW = N / 16;
  pl.col_blocks = (int)((NW + 63) / 64);
  const int64_t T = K / 32;
  int64_t rows_cap = (int64_t)(kGemvScaleGroups - 1) * group_size;
  if (rows_cap > kGemvRowsPerBlock) rows_cap = kGemvRowsPerBlock;
  const int64_t tiles_max = rows_cap / 32 > 0 ? rows_cap / 32 : 1;
  const int64_t min_splits = (T + tiles_max - 1) / tiles_max;
  const int64_t target = kTargetBlocks * gemv_blocks_per_cu(M == 1 ? 1 : 4);
  const int64_t want = target / pl.col_blocks > 0 ? target / pl.col_blocks : 1;
  int64_t max_splits = T / 2;  // at least two 8-row tiles per wave
  if (max_splits < 1) max_splits = 1;
  int64_t splits = want < max_splits ? want : max_splits;
  if (splits < min_splits) splits = min_splits;
  int64_t tps = (T + splits - 1) / splits;
  if (tps < 1) tps = 1;
  splits = (T + tps - 1) / tps;
  pl.splits = (int)splits;
  pl.tiles_per_split = (int)tps;
  pl.workspace = splits > 1 ? (size_t)(splits * M * N * (int64_t)sizeof(float)) : 0;
  return pl;
}

template <typename DT, int MR, int Z>
static void launch_gemv_t(const DecodeParams& p, const DecodePlan& pl, bool dense, hipStream_t st) {
  const dim3 grid(pl.col_blocks, pl.splits);
  if (dense)
    launch_main_kernel(gemv_kernel<DT, MR, Z, true>, grid, dim3(256), st, p);
  else
    launch_main_kernel(gemv_kernel<DT, MR, Z, false>, grid, dim3(256), st, p);
}

template <typename DT, int MR>
static int launch_gemv_mr(const DecodeParams& p, const DecodePlan& pl, int Z, bool dense, hipStream_t st) {
  switch (Z) {
    case 1: launch_gemv_t<DT, MR, 1>(p, pl, dense, st); break;
    case 2: launch_gemv_t<DT, MR, 2>(p, pl, dense, st); break;
    case 3: launch_gemv_t<DT, MR, 3>(p, pl, dense, st); break;
    case 4: launch_gemv_t<DT, MR, 4>(p, pl, dense, st); break;
    default: return GRINQH_ERR_INVALID;
  }
  return GRINQH_OK;
}

template <typename DT>
static int launch_gemv_dt(const DecodeParams& p, const DecodePlan& pl, int Z, bool dense, hipStream_t st) {
  return p.M == 1 ? launch_gemv_mr<DT, 1>(p, pl, Z, dense, st) : launch_gemv_mr<DT, 4>(p, pl, Z, dense, st);
}

int launch_gemv(const DecodeParams& p, const DecodePlan& pl, int max_bits, int dtype, bool dense, hipStream_t st) {
  if (p.M < 1 || p.M > kGemvMaxRows) return GRINQH_ERR_INVALID;
  const int Z = max_bits / 2;
  const int rc = dtype == GRINQH_DTYPE_BF16 ? launch_gemv_dt<BF16>(p, pl, Z, dense, st)
                                            : launch_gemv_dt<F16>(p, pl, Z, dense, st);
  if (rc != GRINQH_OK) return rc;
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
