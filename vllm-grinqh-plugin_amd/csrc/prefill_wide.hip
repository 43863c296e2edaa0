// Large-batch fp16 prefill GRINQH product without a dense weight: a
// dequantize-into-LDS GEMM with 256 x 256 output tiles on
// v_mfma_f32_32x32x16_f16.  It computes what the reference's
// dequantize-then-matmul split does (grinqh/kernel.py:561-587: Wd = RNE(W * s)
// in the activation dtype, X @ Wd with fp32 accumulation; graded batches
// RNE(w_eff * s)) and serves the products that may not allocate the dense
// weight (the allocation-free entry point).  With a workspace the library
// path (dense weight written once, then the library GEMM) is faster on this
// hardware: one wave per SIMD (the 256 accumulators of a 128 x 128 wave tile
// fill the accumulation registers) issues the dequantization, the plane and
// x loads and the LDS traffic besides its MFMAs, and keeps the matrix cores
// busy about a third of the time.
//
// Block: 256 threads, four waves as 2 x 2, each wave 128 rows x 128 logical
// columns (4 x 4 MFMA tiles of 32 x 32).  The block's 256 columns are 16
// plane-word columns w0..w0+15 times the 16 column tiles their words carry
// (tile r = columns r*NW + w0 .. r*NW + w0 + 15).  A stage is 64 rows of K;
// per stage each wave runs 16 groups of 4 MFMAs and, between them, reads the
// A fragments two groups ahead and the next k step's B fragments, and does
// one piece of the next stage: writes x as is and the weight as RNE(w * s)
// (graded: the row's inactive planes masked, its midpoint bias added) into
// the LDS buffer the MFMAs are not reading, and issues the global loads of
// the stage after it (x 256 x 64 halves, 64 rows x Z planes x 16 words,
// scales) once their registers are free.
// LDS tiles are rows of 64 halves (128 bytes): 16-byte chunk ch of row r is
// stored at chunk position ch ^ (r & 7), so that the eight lanes one LDS
// cycle serves (fragment reads: eight rows of one chunk; stores: one row's
// eight chunks, or eight columns of one chunk) touch eight different banks.
#include <type_traits>

#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

namespace {

constexpr int kWideBM = 256;  // rows per block
constexpr int kWideBK = 64;   // K rows per stage
// Row blocks per group of the block order: consecutive blocks (which an XCD
// runs together, see xcd_chunked) share the x rows of one group and the
// plane columns of a few column blocks, so both are fetched into that XCD's
// L2 once.
constexpr int kWideGroupRows = 8;

// Half index of (row, 16-byte chunk) in a swizzled LDS tile of 64-half rows.
__device__ __forceinline__ int swz(int row, int chunk) { return row * 64 + ((chunk ^ (row & 7)) << 3); }

typedef float f32x16_t __attribute__((ext_vector_type(16)));
__device__ __forceinline__ f32x16_t mfma32x32x16_f16(const u32x4_t& a, const u32x4_t& b, f32x16_t c) {
  return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c, 0,
                                                0, 0);
}

}  // namespace

template <int Z, bool DENSE>
__global__ __launch_bounds__(256, 1) void prefill_wide_kernel(PrefillParams p) {
  using DT = F16;
  constexpr int BM = kWideBM, BK = kWideBK, NT = 256;
  constexpr int SH = 8 - 2 * Z;
  __shared__ __align__(16) uint16_t s_a[2][BM * BK];
  __shared__ __align__(16) uint16_t s_b[2][256 * BK];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int c = lane & 15, q = lane >> 4;

  // block order: groups of kWideGroupRows row blocks whose tiles are
  // numbered row block fastest
  const int col_blocks = p.NW / 16, row_blocks = (p.M + BM - 1) / BM;
  const int t = xcd_chunked(blockIdx.x, gridDim.x);
  const int group = t / (kWideGroupRows * col_blocks);
  const int first_rb = group * kWideGroupRows;
  const int group_rows = min(row_blocks - first_rb, kWideGroupRows);
  const int t_in = t - group * kWideGroupRows * col_blocks;
  const int rb = first_rb + t_in % group_rows, cb = t_in / group_rows;
  const int w0 = cb * 16, m0 = rb * BM;
  const int s_begin = 0, s_end = p.K / BK;  // the whole K range

  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.x), (short)0, (int)((uint64_t)p.M * p.ldx * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.planes), (short)0, (int)((uint64_t)p.K * (uint32_t)(Z * p.NW) * 4u), 0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.scale), (short)0, (int)((uint64_t)((p.K + p.gs - 1) / p.gs) * p.N * 2u), 0x00020000);

  // dequantizing roles: word column wcol, rows 8*rg8 .. 8*rg8+7 of the stage,
  // column tiles 8*rh .. 8*rh+7 (rh is uniform over a wave)
  const int wcol = tid & 15, rg8 = (tid >> 4) & 7;
  const int rh = __builtin_amdgcn_readfirstlane(tid >> 7);
  const uint32_t plane_row_bytes = (uint32_t)(Z * p.NW) * 4u;
  const uint32_t p_col_off = (uint32_t)(w0 + wcol) * 4u;
  const uint32_t s_col_off = ((uint32_t)(8 * rh) * (uint32_t)p.NW + (uint32_t)(w0 + wcol)) * 2u;

  // Graded fp16 overflow guard: RNE(w_eff * s) overflows where
  // |w_eff| * |s| > 65504 (|w_eff| <= 2^(2Z-1)), which the reference's fp32
  // products do not.  A block whose scales (its K range, its 256 columns)
  // reach past kScaleLimit builds B from s * 2^-e and scales its sums by 2^e.
  constexpr bool GUARD = !DENSE;
  constexpr uint32_t kScaleLimit = 0x7BFFu - ((uint32_t)(2 * Z - 1) << 10);  // 65504 / 2^(2Z-1), fp16 bits
  int up_exp = 0;
  if constexpr (GUARD) {
    __shared__ uint32_t s_wmax[4];
    const int g_lo = (s_begin * BK) / p.gs, g_hi = (s_end * BK - 1) / p.gs;
    const int total = (g_hi - g_lo + 1) * 256;  // (group, column tile, word column)
    uint32_t hm = 0;
    for (int i0 = tid; i0 < total; i0 += NT * 8) {
      uint16_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = i0 + NT * u;
        const int col = ((idx >> 4) & 15) * p.NW + w0 + (idx & 15);
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
    for (int w = 0; w < 4; ++w) hm = max(hm, s_wmax[w]);
    if (hm > kScaleLimit) up_exp = (int)(hm >> 10) - (int)(kScaleLimit >> 10);
  }
  const float down_scale = __builtin_ldexpf(1.f, -up_exp), up_scale = __builtin_ldexpf(1.f, up_exp);

  // registers of one stage's global loads
  struct Slot {
    u32x4_t xa[8];
    uint32_t D[8][Z];
    float sig[8];
    uint16_t sraw[8];
  };
  // Loads: the stage moves the lane offset (one VALU add per family), the
  // scalar offsets are loop invariant.  x: lane row m0 + tid / 8, chunk
  // tid % 8, piece i 32 rows further down.  Rows past M must load 0, so the
  // whole offset of an x piece goes in the vector offset, the part the
  // buffer's range check certainly covers (the scalar offset is not relied
  // on for it); prefill_wide_applies bounds (M + 256) * ldx * 2 below 2^31,
  // so no offset wraps.
  const uint32_t x_lane_off = (uint32_t)(((int64_t)(m0 + (tid >> 3)) * p.ldx + 8 * (tid & 7)) * 2);
  uint32_t x_piece_off[8];  // wave-uniform
#pragma unroll
  for (int i = 0; i < 8; ++i) x_piece_off[i] = (uint32_t)i * (uint32_t)(32 * p.ldx * 2);
  auto load_x = [&](int s, Slot& S) {
    const uint32_t voff = x_lane_off + (uint32_t)(s * BK * 2);
#pragma unroll
    for (int i = 0; i < 8; ++i)
      S.xa[i] = __builtin_bit_cast(
          u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(voff + x_piece_off[i]), 0, 0));
  };
  // planes: lane rows 8*rg8.. of the stage, word column w0 + wcol; row e and
  // plane z by scalar offset
  const uint32_t p_lane_off = (uint32_t)(8 * rg8) * plane_row_bytes + p_col_off;
  uint32_t p_soff[8][Z];
#pragma unroll
  for (int e = 0; e < 8; ++e)
#pragma unroll
    for (int z = 0; z < Z; ++z) p_soff[e][z] = (uint32_t)e * plane_row_bytes + (uint32_t)z * p.NW * 4u;
  // scales: the group's row by lane offset, column tile r by scalar offset
  uint32_t s_soff[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) s_soff[r] = (uint32_t)r * p.NW * 2u;
  auto load_w = [&](int s, Slot& S) {
    const int k0 = s * BK;
    const uint32_t voff = p_lane_off + (uint32_t)k0 * plane_row_bytes;
#pragma unroll
    for (int e = 0; e < 8; ++e)
#pragma unroll
      for (int z = 0; z < Z; ++z)
        S.D[e][z] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(prsrc, (int)voff, (int)p_soff[e][z], 0);
    if constexpr (!DENSE) {
      const f32x4_t* sg = reinterpret_cast<const f32x4_t*>(p.sigma + k0 + 8 * rg8);
      const f32x4_t s0 = sg[0], s1 = sg[1];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        S.sig[e] = s0[e];
        S.sig[4 + e] = s1[e];
      }
    }
    const uint32_t svoff = s_col_off + (uint32_t)(k0 / p.gs) * (uint32_t)p.N * 2u;
#pragma unroll
    for (int r = 0; r < 8; ++r) S.sraw[r] = __builtin_amdgcn_raw_buffer_load_b16(srsrc, (int)svoff, (int)s_soff[r], 0);
  };

  // Pieces of one stage's LDS stores: x rows as they are (two 16-byte chunks
  // per piece), and the weight graded (union), rebuilt into code bytes and
  // dequantized to RNE(w * s), eight rows of one column per 16-byte store.
  auto store_x = [&](int buf, const Slot& S, int i) {
    const int h = tid + NT * i, row = h >> 3, piece = h & 7;
    *reinterpret_cast<u32x4_t*>(&s_a[buf][swz(row, piece)]) = S.xa[i];
  };
  uint32_t negc[4], s2[8], V[8];
  auto prepare_w = [&](Slot& S) {
    int beta[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const uint32_t bits = DENSE ? ((1u << Z) - 1u) : zone_bits<Z>(S.sig[e], p.thr.t);
      beta[e] = DENSE ? 0 : midpoint_bias<Z>(bits);
      if constexpr (!DENSE) {
#pragma unroll
        for (int z = 0; z < Z; ++z) S.D[e][z] &= 0u - ((bits >> z) & 1u);
      }
    }
    uint32_t xm[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) xm[e] = 0xAAAAAAAAu;  // offset binary: u = int8(U & mask) + 128
    prepare_planes<Z, 8>(S.D, xm);
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
      const uint16_t c0 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[2 * pp]));
      const uint16_t c1 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[2 * pp + 1]));
      negc[pp] = (uint32_t)c0 | ((uint32_t)c1 << 16);
    }
#pragma unroll
    for (int r = 0; r < 8; ++r) {
      const uint16_t sh = (GUARD && up_exp > 0) ? from_f32<DT>(to_f32<DT>(S.sraw[r]) * down_scale) : S.sraw[r];
      s2[r] = (uint32_t)sh | ((uint32_t)sh << 16);
    }
  };
  auto store_w = [&](int buf, int jj, int b) {  // column tile 8*rh + 4*jj + b from V (code dwords of j = 2*rh + jj)
    const int r = 4 * jj + b;
    u32x4_t w;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) w[pp] = Dequant<F16, SH>::pair(V[2 * pp], V[2 * pp + 1], b, negc[pp], s2[r]);
    *reinterpret_cast<u32x4_t*>(&s_b[buf][swz((8 * rh + r) * 16 + wcol, rg8)]) = w;
  };

  f32x16_t acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[i][t] = (f32x16_t)0.f;

  // MFMA operands (v_mfma_f32_32x32x16_f16: lane l holds row / column l % 32,
  // k = 8 * (l / 32) .. +7 of the 16-deep k step): B fragments of two k steps
  // (four 32-column tiles each: column tiles 8*wn + 2t, +1), A fragments in a
  // ring of four (read two groups ahead)
  u32x4_t Bf[2][4], Af[4];
  const int l32 = lane & 31, kh = lane >> 5;
  auto read_b = [&](int buf, int ks, u32x4_t (&B)[4]) {
#pragma unroll
    for (int t = 0; t < 4; ++t)
      B[t] = *reinterpret_cast<const u32x4_t*>(&s_b[buf][swz((8 * wn + 2 * t) * 16 + l32, 2 * ks + kh)]);
  };
  auto read_a = [&](int buf, int g) {  // group g: k step g / 4, row tile g % 4
    return *reinterpret_cast<const u32x4_t*>(&s_a[buf][swz(wm * 128 + 32 * (g & 3) + l32, 2 * (g >> 2) + kh)]);
  };
  auto mfma_group = [&](int g) {
#pragma unroll
    for (int t = 0; t < 4; ++t) acc[g & 3][t] = mfma32x32x16_f16(Af[g & 3], Bf[(g >> 2) & 1][t], acc[g & 3][t]);
  };
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // A stage is 16 groups of 4 MFMAs (group g: k step g / 4, row tile g % 4).
  // Around group g: the A fragment of group g+2 is read, and one piece of the
  // next stage's work runs (its x stores, grading, code dwords, weight
  // stores; the loads of the stage after it once their registers are free).
  // All stores are done by group 13; the barrier follows it, and the next
  // stage's first fragments are read while groups 14 and 15 multiply.
  // Loads past the range repeat its last stage and are never stored
  // (unconditional loads keep the wait counts exact).
  Slot S;
  const int last = s_end - 1;
  load_x(s_begin, S);
  load_w(s_begin, S);
#pragma unroll
  for (int i = 0; i < 8; ++i) store_x(0, S, i);
  prepare_w(S);
#pragma unroll
  for (int jj = 0; jj < 2; ++jj) {
    code_dwords<Z, 8>(S.D, 2 * rh + jj, V);
#pragma unroll
    for (int b = 0; b < 4; ++b) store_w(0, jj, b);
  }
  load_x(min(s_begin + 1, last), S);
  load_w(min(s_begin + 1, last), S);
  barrier();
  read_b(0, 0, Bf[0]);
  Af[0] = read_a(0, 0);
  Af[1] = read_a(0, 1);
  // one stage: MORE (compile time) when a next stage is to be stored
  auto run_stage = [&](int s, auto more_tag) {
    constexpr bool more = decltype(more_tag)::value;
    const int buf = (s - s_begin) & 1, nb = buf ^ 1;
#pragma unroll
    for (int g = 0; g < 16; ++g) {
      if (g + 2 < 16) Af[(g + 2) & 3] = read_a(buf, g + 2);
      if ((g & 3) == 1 && g < 12) read_b(buf, (g >> 2) + 1, Bf[((g >> 2) + 1) & 1]);
      if constexpr (more) {
        if (g < 4) {
          store_x(nb, S, 2 * g);
          store_x(nb, S, 2 * g + 1);
          if (g == 3) load_x(min(s + 2, last), S);
        } else if (g == 4) {
          prepare_w(S);
        } else if (g == 5 || g == 10) {
          code_dwords<Z, 8>(S.D, 2 * rh + (g == 10 ? 1 : 0), V);
          if (g == 10) load_w(min(s + 2, last), S);
        } else if (g >= 6 && g <= 9) {
          store_w(nb, 0, g - 6);
        } else if (g == 11) {
          store_w(nb, 1, 0);
          store_w(nb, 1, 1);
        } else if (g == 12 || g == 13) {
          store_w(nb, 1, g - 10);
        }
      }
      if (g == 14) {
        barrier();
        if constexpr (more) {
          read_b(nb, 0, Bf[0]);
          Af[0] = read_a(nb, 0);
          Af[1] = read_a(nb, 1);
        }
      }
      mfma_group(g);
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  for (int s = s_begin; s < last; ++s) run_stage(s, std::true_type{});
  run_stage(last, std::false_type{});

  // epilogue: lane l holds column l % 32 of each 32 x 32 tile, rows
  // 8 * (v / 4) + 4 * (l / 32) + v % 4 for its accumulators v
#pragma unroll
  for (int i = 0; i < 4; ++i)
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      const int64_t n = (int64_t)(8 * wn + 2 * t + (l32 >> 4)) * p.NW + w0 + (lane & 15);
#pragma unroll
      for (int v = 0; v < 16; ++v) {
        const int m = m0 + wm * 128 + 32 * i + 8 * (v >> 2) + 4 * kh + (v & 3);
        if (m >= p.M) continue;
        const float y = DENSE ? acc[i][t][v] : graded_nonfinite_to_nan(acc[i][t][v] * up_scale);
        p.y[(int64_t)m * p.N + n] = finish_output<DT>(y, p.bias, (int)n);
      }
    }
}

bool prefill_wide_applies(int64_t M, int64_t K, int64_t N, int64_t ldx, int gs, int dtype) {
  // x offsets of the last row block stay below 2^31 even for rows past M
  if (dtype != GRINQH_DTYPE_F16 || M < kWidePrefillRows || N % 256 != 0 || K % kWideBK != 0 || gs % kWideBK != 0 ||
      (M + kWideBM) * ldx * 2 >= ((int64_t)1 << 31))
    return false;
  return (N / 256) * ((M + kWideBM - 1) / kWideBM) >= kWideMinTiles;
}

template <int Z>
static void launch_wide_z(const PrefillParams& p, bool dense, hipStream_t st) {
  const dim3 grid((p.NW / 16) * ((p.M + kWideBM - 1) / kWideBM));
  if (dense)
    launch_main_kernel(prefill_wide_kernel<Z, true>, grid, dim3(256), st, p);
  else
    launch_main_kernel(prefill_wide_kernel<Z, false>, grid, dim3(256), st, p);
}

int launch_prefill_wide(const PrefillParams& p, int max_bits, bool dense, hipStream_t st) {
  if (!dense && p.sigma == nullptr) return GRINQH_ERR_INVALID;
  if (!prefill_wide_applies(p.M, p.K, p.N, p.ldx, p.gs, GRINQH_DTYPE_F16)) return GRINQH_ERR_INVALID;
  switch (max_bits / 2) {
    case 1: launch_wide_z<1>(p, dense, st); break;
    case 2: launch_wide_z<2>(p, dense, st); break;
    case 3: launch_wide_z<3>(p, dense, st); break;
    case 4: launch_wide_z<4>(p, dense, st); break;
    default: return GRINQH_ERR_INVALID;
  }
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
