// Large-batch GRINQH prefill: a dequantize-into-LDS GEMM on
// v_mfma_f32_16x16x32_{f16,bf16} with tall block tiles.
//
// Computes what the reference's dequantize-then-matmul split computes
// (grinqh_prefill_gemm_compiled, grinqh/kernel.py:561-587: Wd = RNE(W * s)
// in the activation dtype, X @ Wd with fp32 accumulation, then the bias add
// of :706-708), and in union mode the same with RNE(w_eff * s) from the batch
// statistic (the grade of grinqh/kernel.py:249-289), without writing the
// dense weight.
//
// Block: four waves, one per SIMD (all 512 registers of a lane: the
// accumulators stay in AGPRs, updated in place), block tile 64 * RT rows x
// 128 logical columns (RT = 8: 512 rows, or 4: 256 rows), each wave a
// (16 RT) x 128 tile of 16 x 16 MFMA tiles.  The 128 columns are 8
// plane-word columns w0..w0+7 times the 16 column tiles their words carry:
// block column bc = 8 r + wc is logical column r * NW + w0 + wc.  The waves
// share the weight and nothing else, so
//   * x (the A operand) is repacked first (repack_x_kernel) into 1 KiB MFMA
//     fragments and goes from global memory (L2) straight into each wave's
//     registers, one contiguous 16-byte load per lane and fragment, half a
//     stage ahead or more;
//   * the weight is dequantized once per block per 64-row stage into LDS
//     (RNE(w * s) in the activation dtype, [column][k] with k contiguous) and
//     read back as B fragments by every wave -- each dequantized weight feeds
//     64 * RT rows.
// The dequantization is spread over the MFMA groups of the previous stage: a
// producer thread owns one word column and two rows of a stage (all Z planes,
// loaded 1.5 stages ahead) and writes 16 column tiles of 2 k values each.
// The MFMAs take the weight as their first operand, so each lane ends with
// four consecutive columns of one row: 8-byte output stores.  Nothing in the
// MFMA loop branches.
//
// Split over K (grid.y): the ranges of an output tile store fp32 partial sums
// and count themselves done on the tile's counter; the range that arrives
// last adds all ranges in range order (the result does not depend on which
// finished last), casts, adds the bias and clears the counter.
#include <type_traits>
#include <utility>

#include "grinqh_common.h"
#include "grinqh_launch.h"
#include "splitk_complete.h"

namespace grinqh {

namespace {

constexpr int kTallBK = 64;         // K rows per stage
constexpr int kTallWords = 8;       // plane-word columns per block (128 logical columns)

typedef float f32x2_t __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));

// Half index of (block column, 16-byte k chunk) in the LDS weight tile: rows
// of 64 halves (128 bytes), chunk ch of column c at chunk position
// ch ^ (c & 7).  The LDS serves 128 bytes (32 four-byte banks) per cycle, so
// both access patterns are conflict-free: a fragment read (eight consecutive
// columns, one chunk, 16 bytes each) hits eight different chunk positions,
// and a producer store (eight columns 8 r .. 8 r + 7 times four row pairs,
// 4 bytes each) sends the eight columns to eight chunk positions.
__device__ __forceinline__ int bswz(int col, int chunk) { return col * 64 + ((chunk ^ (col & 7)) << 3); }

// Two k values (rows e0, e1: low and high half) of column tile beta as
// RNE(w * s) in bf16: u is the offset-binary code byte, c_row = 128 -
// beta_row * 2^sh, s_sh = s * 2^-sh, so (u - c_row) * s_sh = w_eff * s exactly
// in fp32 (at most 17 significant bits), rounded once to bf16.
__device__ __forceinline__ uint32_t bf16_pair(uint32_t V0, uint32_t V1, int beta, float c0, float c1, float s_sh) {
  const float a = ((float)((V0 >> (8 * beta)) & 0xFFu) - c0) * s_sh;
  const float b = ((float)((V1 >> (8 * beta)) & 0xFFu) - c1) * s_sh;
  return __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2_t){a, b}, bf16x2_t));
}

// f(integral_constant<int, 0>) ... f(integral_constant<int, N - 1>): the
// group index of a stage must be a compile-time constant (a runtime index
// would address the accumulators dynamically), and #pragma unroll gives up on
// the largest stage bodies
template <typename F, int... I>
__device__ __forceinline__ void static_for_impl(F&& f, std::integer_sequence<int, I...>) {
  (f(std::integral_constant<int, I>{}), ...);
}
template <int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  static_for_impl(f, std::make_integer_sequence<int, N>{});
}

}  // namespace

template <typename DT, int Z, bool DENSE, int RT>
__global__ __launch_bounds__(256, 1) void prefill_tall_kernel(PrefillParams p) {
  static_assert(RT == 8 || RT == 4, "512- or 256-row blocks");
  constexpr int MW = 4;  // waves: one per SIMD
  constexpr int NT = 64 * MW;
  constexpr int BK = kTallBK;
  constexpr int BM = 16 * RT * MW;
  constexpr int SH = 8 - 2 * Z;
  constexpr bool IS_F16 = DT::id == F16::id;
  __shared__ __align__(16) uint16_t s_b[2][128 * BK];
  __shared__ __align__(16) uint16_t s_scale[2][8 * 16];  // [stage parity][word column][column tile]

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int l16 = lane & 15, kq = lane >> 4;

  // ---- work item: blocks renumbered so that each XCD runs consecutive items
  // (shared weight columns and x rows meet in one L2); items below dp_tiles
  // are whole tiles, the rest the K ranges of the split tiles, range fastest.
  // Tile order: groups of GR row blocks, row block fastest.  512-row blocks
  // take one row block per group (the columns run fastest): the tiles an
  // XCD runs at the same time read the same rows of x, which its L2 then
  // serves, and each weight tile comes back for the other row blocks from
  // the memory side; at 2048 rows (dense, kernel time) gate_up took 532 ->
  // 499 us and down 280 -> 267 us against groups of four.  256-row blocks
  // (half the x per row block) keep groups of four, the weight shared by four
  // row blocks on one XCD: down at 2048 rows without a workspace (eight row
  // blocks, weights cold) 308 us against 320-332 us with one per group.
  constexpr int GR = RT == 8 ? 1 : 4;
  const int col_blocks = p.NW / kTallWords, row_blocks = (p.M + BM - 1) / BM;
  const int item = xcd_chunked(blockIdx.x, gridDim.x);
  const bool whole = item < p.dp_tiles;
  const int jt = whole ? 0 : (item - p.dp_tiles) / p.splits;  // index among the split tiles
  const int t = whole ? item : p.dp_tiles + jt;
  const int split = whole ? 0 : (item - p.dp_tiles) - jt * p.splits;
  const int splits = whole ? 1 : p.splits;
  const int group = t / (GR * col_blocks);
  const int first_rb = group * GR;
  const int group_rows = min(row_blocks - first_rb, GR);
  const int t_in = t - group * GR * col_blocks;
  const int rb = first_rb + t_in % group_rows, cb = t_in / group_rows;
  const int w0 = cb * kTallWords, m0 = rb * BM;
  const int stages = p.K / BK;
  const int s_begin = (int)((int64_t)stages * split / splits);
  const int s_end = (int)((int64_t)stages * (split + 1) / splits);
  const int last = s_end - 1;

  // ---- x, repacked by repack_x_kernel into 1 KiB fragments (one operand of
  // v_mfma_f32_16x16x32 each: 16 rows x 32 k, lane order), fragment (row tile
  // T, k step kk) at ((T * K / 32) + kk) KiB: every load reads one contiguous
  // KiB.  The descriptor ends after the last row tile, so tiles past the
  // batch read 0; the tile is part of the vector offset (range checked), the
  // k step the scalar offset
  const int row0 = __builtin_amdgcn_readfirstlane(m0 + 16 * RT * wave);
  const int rows_valid = __builtin_amdgcn_readfirstlane(max(0, min(p.M - row0, 16 * RT)));
  const uint32_t kfrags = (uint32_t)(p.K / 32);
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.x), (short)0, (int)((uint32_t)((p.M + 15) / 16) * kfrags * 1024u), 0x00020000);
  const uint32_t a_voff = ((uint32_t)(row0 / 16) * kfrags) * 1024u + (uint32_t)lane * 16u;

  // ---- producer role (every thread): word column wc, row pair rp0 of a
  // stage, all 16 column tiles; scale loader role: column tile
  // sr = (tid / 8) % 16, word column wc
  const int wc = tid & 7, rp0 = tid >> 3;
  const uint32_t row_bytes = (uint32_t)(Z * p.NW) * 4u;
  const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.planes), (short)0, (int)((uint64_t)p.K * row_bytes), 0x00020000);
  const __amdgpu_buffer_rsrc_t srsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.scale), (short)0, (int)((uint64_t)((p.K + p.gs - 1) / p.gs) * p.N * 2u), 0x00020000);
  // plane word (row 2 rp0 of the stage, plane 0, word column w0 + wc); the
  // pair's second row, the plane and the stage go in the scalar offset (every
  // plane row lies inside the array)
  const uint32_t p_voff = (uint32_t)(2 * rp0) * row_bytes + (uint32_t)(w0 + wc) * 4u;
  const int sr = (tid >> 3) & 15;
  const uint32_t s_voff = ((uint32_t)sr * (uint32_t)p.NW + (uint32_t)(w0 + wc)) * 2u;

  // Graded fp16 overflow guard: RNE(w_eff * s) overflows where
  // |w_eff| * |s| > 65504 (|w_eff| <= 2^(2Z-1)), which the reference's fp32
  // products do not.  A block whose scales (its K range, its 128 columns)
  // reach past kScaleLimit builds B from s * 2^-e and scales its sums by 2^e.
  constexpr bool GUARD = !DENSE && IS_F16;
  constexpr uint32_t kScaleLimit = 0x7BFFu - ((uint32_t)(2 * Z - 1) << 10);  // 65504 / 2^(2Z-1), fp16 bits
  int up_exp = 0;
  if constexpr (GUARD) {
    __shared__ uint32_t s_wmax[MW];
    const int g_lo = (s_begin * BK) / p.gs, g_hi = (s_end * BK - 1) / p.gs;
    const int total = (g_hi - g_lo + 1) * 128;  // (group, column tile, word column)
    uint32_t hm = 0;
    for (int i0 = tid; i0 < total; i0 += NT * 8) {
      uint16_t v[8];
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const int idx = i0 + NT * u;
        const int col = ((idx >> 3) & 15) * p.NW + w0 + (idx & 7);
        const uint32_t off = idx < total ? ((uint32_t)(g_lo + (idx >> 7)) * (uint32_t)p.N + (uint32_t)col) * 2u
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
    for (int w = 0; w < MW; ++w) hm = max(hm, s_wmax[w]);
    if (hm > kScaleLimit) up_exp = (int)(hm >> 10) - (int)(kScaleLimit >> 10);
  }
  const float down_scale = __builtin_ldexpf(1.f, -up_exp), up_scale = __builtin_ldexpf(1.f, up_exp);

  // ---- registers of one stage's weight loads (planes and, graded, the two
  // rows' grade words, loaded one stage ahead of their dequantization) and the
  // scale of the stage two ahead on its way to the LDS ring s_scale
  uint32_t D[2][Z];
  u32x2_t gw;
  uint16_t sc_in = 0;
  auto load_planes = [&](int s) {
    const uint32_t k0 = (uint32_t)(s * BK);
#pragma unroll
    for (int e = 0; e < 2; ++e)
#pragma unroll
      for (int z = 0; z < Z; ++z)
        D[e][z] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(
            prsrc, (int)p_voff, (int)((k0 + (uint32_t)e) * row_bytes + (uint32_t)z * p.NW * 4u), 0);
    if constexpr (!DENSE) gw = *reinterpret_cast<const u32x2_t*>(p.grades + k0 + 2 * rp0);
  };
  auto load_scale = [&](int s) {
    // the division is done on the vector unit; readfirstlane keeps the offset
    // scalar (a vector soffset would make the compiler loop over lanes)
    const int soff = __builtin_amdgcn_readfirstlane((int)(((uint32_t)(s * BK) / (uint32_t)p.gs) * (uint32_t)p.N * 2u));
    sc_in = __builtin_amdgcn_raw_buffer_load_b16(srsrc, (int)s_voff, soff, 0);
  };
  // every thread stores the scale it loaded: the threads of one (sr, wc)
  // loaded the same element, and no branch splits the MFMA loop.  The
  // overflow guard's factor is applied here, once per scale (unconditionally:
  // exact when up_exp == 0), rather than to every scale a producer reads.
  auto store_scale = [&](int slot) {
    uint16_t v = sc_in;
    if constexpr (GUARD) v = from_f32<DT>(to_f32<DT>(v) * down_scale);
    s_scale[slot][wc * 16 + sr] = v;
  };

  // ---- dequantization of one stage: prep grades the rows, flips and rotates
  // the planes and rebuilds all code dwords (V, so the plane registers are
  // free for the next stage's loads right away) and takes this word column's
  // 16 scales from the ring; then 16 column tiles of 4-byte stores
  uint32_t V[4][2];
  uint32_t negc;  // fp16: (-c_row) of the pair's two rows
  f32x2_t cbf;    // bf16: c_row of the two rows
  uint32_t s2[8];  // this word column's 16 scales (tiles 2 q, 2 q + 1), as loaded
  // prep in pieces: grade (zone masks and the row constants, from the rows'
  // grade words when graded; the offset-binary flip and plane rotation), code
  // dwords of each group of four column tiles, scales
  auto prep_grade = [&]() {
    if constexpr (!DENSE) {
#pragma unroll
      for (int e = 0; e < 2; ++e)
#pragma unroll
        for (int z = 0; z < Z; ++z) D[e][z] &= 0u - ((gw[e] >> (16 + z)) & 1u);
    }
    const uint32_t xm[2] = {0xAAAAAAAAu, 0xAAAAAAAAu};  // offset binary: u = int8(U & mask) + 128
    prepare_planes<Z, 2>(D, xm);
    if constexpr (IS_F16) {
      if constexpr (DENSE) {
        const uint32_t c = f32_to_f16_bits(-(float)(1024 + (128 >> SH)));
        negc = c | (c << 16);
      } else {
        negc = (gw[0] & 0xFFFFu) | (gw[1] << 16);
      }
    } else {
      if constexpr (DENSE)
        cbf = f32x2_t{128.f, 128.f};
      else
        cbf = f32x2_t{(float)(int16_t)(gw[0] & 0xFFFFu), (float)(int16_t)(gw[1] & 0xFFFFu)};
    }
  };
  auto prep_code = [&](int j) { code_dwords<Z, 2>(D, j, V[j]); };
  auto prep_scales = [&](int sslot) {
#pragma unroll
    for (int c = 0; c < 2; ++c) {
      const u32x4_t sa = *reinterpret_cast<const u32x4_t*>(&s_scale[sslot][wc * 16 + 8 * c]);
#pragma unroll
      for (int q = 0; q < 4; ++q) s2[4 * c + q] = sa[q];
    }
  };
  auto prep = [&](int sslot) {
    prep_grade();
#pragma unroll
    for (int j = 0; j < 4; ++j) prep_code(j);
    prep_scales(sslot);
  };
  // column tile r's scale is half r % 2 of s2[r / 2]: fp16 multiplies by it
  // broadcast (an operand select of the packed multiply), bf16 by s * 2^-sh
  auto store_w = [&](int buf, int r) {  // column tile r = 4 j + b: k = 2 rp0, 2 rp0 + 1 of the stage
    const int j = r >> 2, b = r & 3;
    uint32_t w;
    if constexpr (IS_F16) {
      w = Dequant<F16, SH>::pair_half(V[j][0], V[j][1], b, negc, s2[r >> 1], r & 1);
    } else {
      const float sc = to_f32<DT>((uint16_t)((r & 1) ? (s2[r >> 1] >> 16) : (s2[r >> 1] & 0xFFFFu))) *
                       (1.0f / (float)(1 << SH));
      w = bf16_pair(V[j][0], V[j][1], b, cbf[0], cbf[1], sc);
    }
    *reinterpret_cast<uint32_t*>(&s_b[buf][bswz(8 * r + wc, rp0 >> 2) + 2 * (rp0 & 3)]) = w;
  };

  // ---- MFMA operands (v_mfma_f32_16x16x32): x fragments A[ks][i] (row tile
  // i, k step ks of 32), each reloaded for the next stage right after its
  // last group of MFMAs; weight fragments Bf[tt] (column tile tt) of one k
  // step at a time, each half reloaded four groups before its next use
  u32x4_t A[2][RT];
  u32x4_t Bf[8];
  auto load_a = [&](int s, int ks, int i) {
    A[ks][i] = __builtin_bit_cast(
        u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)(a_voff + (uint32_t)i * kfrags * 1024u),
                                                       (int)((2 * s + ks) * 1024), 0));
  };
  auto read_b = [&](int buf, int ks, int tt) {
    Bf[tt] = *reinterpret_cast<const u32x4_t*>(&s_b[buf][bswz(16 * tt + l16, 4 * ks + kq)]);
  };
  // written first by the first stage's k step 0 MFMAs (zero C input): a
  // loop entered with the same zero for every accumulator got them
  // reassigned from stage to stage and partly moved through VGPRs
  f32x4_t acc[RT][8];
  auto barrier = [] { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); };

  // ---- one stage: 4 RT groups of four MFMAs, in four phases of RT groups
  // (phase (ks, h): k step ks, column half h; group g = RT * (2 ks + h) + i:
  // row tile i, column tiles 4 h .. 4 h + 3), each group followed by the
  // next stage's load of the x fragment that it was the last to use.  Weight
  // fragments, one phase ahead: the k step 0 half 1 tiles at phase (0, 0)
  // (from this stage's buffer), k step 1 at phases (0, 1) and (1, 0), the
  // next stage's k step 0 half 0 after the barrier, which opens phase (1, 1).
  // The dequantization of the next stage into the other LDS buffer is spread
  // over the groups before the barrier in pieces of similar size: grading,
  // code dwords (then the plane loads of the stage after it, their registers
  // free), scales, 16 column tiles of stores, and the scale of the stage
  // after next into the ring.  Loads past the range repeat its last stage
  // (never used), so the wait counts stay static.
  constexpr int G = 4 * RT;                  // groups per stage
  constexpr int kStoreGroups = 3 * RT - 4;   // groups 3 .. 3 RT - 2 store the 16 column tiles
  auto run_stage = [&](int o, auto more_tag, auto first_tag) {
    constexpr bool more = decltype(more_tag)::value;
    constexpr bool first = decltype(first_tag)::value;
    const int s = s_begin + o;
    const int buf = o & 1, nb = buf ^ 1;
    static_for<G>([&](auto gc) {
      constexpr int g = decltype(gc)::value;
      constexpr int ks = g / (2 * RT), h = (g / RT) & 1, i = g % RT;
      if constexpr (g == 0) {
#pragma unroll
        for (int tt = 4; tt < 8; ++tt) read_b(buf, 0, tt);
      } else if constexpr (g == RT || g == 2 * RT) {
#pragma unroll
        for (int tt = 0; tt < 4; ++tt) read_b(buf, 1, tt + (g == 2 * RT ? 4 : 0));
      }
      if constexpr (more) {
        if constexpr (g == 0) {
          prep_grade();
        } else if constexpr (g == 1) {
          prep_code(0);
          prep_code(1);
        } else if constexpr (g == 2) {
          prep_code(2);
          prep_code(3);
          load_planes(min(s + 2, last));  // the plane registers are free
        } else if constexpr (g < 3 + kStoreGroups) {
          if constexpr (g == 3) prep_scales((o + 1) & 1);
#pragma unroll
          for (int r = (16 * (g - 3)) / kStoreGroups; r < (16 * (g - 2)) / kStoreGroups; ++r) store_w(nb, r);
        } else if constexpr (g == 3 * RT - 1) {
          store_scale(o & 1);  // the scale of stage s + 2 (same parity as s), read in the next stage
          load_scale(min(s + 3, last));
        }
      }
      if constexpr (g == 3 * RT) {
        barrier();
        if constexpr (more) {
#pragma unroll
          for (int tt = 0; tt < 4; ++tt) read_b(nb, 0, tt);
        }
      }
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const int tt = 4 * h + q;
        acc[i][tt] = mfma16x16x32<DT>(Bf[tt], A[ks][i],
                                      (first && ks == 0) ? f32x4_t{0.f, 0.f, 0.f, 0.f} : acc[i][tt]);
      }
      if constexpr (more && h == 1) load_a(s + 1, ks, i);
      __builtin_amdgcn_sched_barrier(0);
    });
  };

  // ---- prologue: stage s_begin into LDS buffer 0; the next stage's planes
  // in flight; scales of the first two stages in the ring, the third's in
  // flight; the first stage's fragments of x; then the stages
  load_scale(s_begin);
  store_scale(0);
  load_scale(min(s_begin + 1, last));
  store_scale(1);
  load_planes(s_begin);
  load_scale(min(s_begin + 2, last));
#pragma unroll
  for (int ks = 0; ks < 2; ++ks)
#pragma unroll
    for (int i = 0; i < RT; ++i) load_a(s_begin, ks, i);
  __syncthreads();  // the scale ring
  prep(0);
  load_planes(min(s_begin + 1, last));
#pragma unroll
  for (int r = 0; r < 16; ++r) store_w(0, r);
  barrier();
#pragma unroll
  for (int tt = 0; tt < 4; ++tt) read_b(0, 0, tt);
  const int S = s_end - s_begin;
  if (S == 1) {
    run_stage(0, std::false_type{}, std::true_type{});
  } else {
    run_stage(0, std::true_type{}, std::true_type{});
    // one stage per iteration: unrolling it further raised the register
    // pressure until the accumulators no longer stayed in place
#pragma clang loop unroll(disable)
    for (int o = 1; o < S - 1; ++o) run_stage(o, std::true_type{}, std::false_type{});
    run_stage(S - 1, std::false_type{}, std::false_type{});
  }

  // ---- epilogue: lane (l16, kq) holds row l16 of each 16 x 16 tile, block
  // columns 16 tt + 4 kq .. + 3 = column tile 2 tt + kq / 2, word columns
  // w0 + 4 (kq % 2) .. + 3: four consecutive logical columns
  auto value = [&](int i, int tt, int v) {
    return DENSE ? acc[i][tt][v] : graded_nonfinite_to_nan(acc[i][tt][v] * up_scale);
  };
  // (columns computed per tile, 32-bit: N < 2^24; the row offset in 64 bits)
  const int ncol0 = (kq >> 1) * p.NW + w0 + 4 * (kq & 1);
  auto ncol = [&](int tt) { return ncol0 + 2 * tt * p.NW; };
  auto elem = [&](int i, int tt) -> int64_t { return (int64_t)(row0 + 16 * i + l16) * p.N + ncol(tt); };
  auto out4 = [&](int i, int tt, f32x4_t a) {  // four outputs of one row: one 8-byte store
    const int n = ncol(tt);
    u32x2_t h;
    h[0] = (uint32_t)finish_output<DT>(a[0], p.bias, n) | ((uint32_t)finish_output<DT>(a[1], p.bias, n + 1) << 16);
    h[1] = (uint32_t)finish_output<DT>(a[2], p.bias, n + 2) | ((uint32_t)finish_output<DT>(a[3], p.bias, n + 3) << 16);
    *reinterpret_cast<u32x2_t*>(&p.y[elem(i, tt)]) = h;
  };
  if (splits == 1) {  // tile by tile (the barrier keeps the accumulator reads from being hoisted)
#pragma unroll
    for (int i = 0; i < RT; ++i)
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) {
        if (16 * i + l16 < rows_valid)
          out4(i, tt, f32x4_t{value(i, tt, 0), value(i, tt, 1), value(i, tt, 2), value(i, tt, 3)});
        __builtin_amdgcn_sched_barrier(0);
      }
    return;
  }
  // split over K: every range stores its partial sums (16-byte agent-scope
  // stores, written through L2; lane-major, one contiguous KiB per store) and,
  // once they have completed, counts itself done on the tile's counter; the
  // range that counts last reads all ranges back and adds them in range order
  // 0, 1, ..., so the result does not depend on which range finished last,
  // then clears the counter for the next launch.  Its accumulators are free
  // by then, which keeps the reduction's registers apart from them.
  constexpr uint32_t kTileBytes = (uint32_t)BM * 128u * 4u;
  const uint32_t part_bytes = (uint32_t)((gridDim.x - (unsigned)p.dp_tiles) / (unsigned)p.splits) *
                              (uint32_t)p.splits * kTileBytes;  // below 2^31: the partial area is capped
  const __amdgpu_buffer_rsrc_t prs = __builtin_amdgcn_make_buffer_rsrc(p.partial, (short)0, (int)part_bytes, 0x00020000);
  auto poff = [&](int i, int tt) { return (uint32_t)(((wave * RT + i) * 8 + tt) * 1024 + lane * 16); };
  auto range_base = [&](int sp) { return (uint32_t)(jt * p.splits + sp) * kTileBytes; };
#pragma unroll
  for (int i = 0; i < RT; ++i)
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      const f32x4_t v{value(i, tt, 0), value(i, tt, 1), value(i, tt, 2), value(i, tt, 3)};
      __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4_t, v), prs, (int)poff(i, tt),
                                             (int)range_base(split), kCpolSc1);
    }
  __shared__ int s_last;
  __builtin_amdgcn_s_waitcnt(0);  // this wave's partial stores have completed
  __syncthreads();
  if (tid == 0) s_last = atomicAdd(&p.counters[jt], 1u) == (unsigned)(splits - 1);
  __syncthreads();
  if (!s_last) return;
  auto load = [&](int sp, int i, int tt) {  // range sp's sums of one row of a 16 x 16 tile
    return __builtin_bit_cast(f32x4_t, __builtin_amdgcn_raw_buffer_load_b128(prs, (int)poff(i, tt),
                                                                              (int)range_base(sp), kCpolSc1));
  };
  // a row tile's eight column tiles of a range in flight at once
#pragma unroll
  for (int i = 0; i < RT; ++i) {
    f32x4_t sum[8];
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) sum[tt] = load(0, i, tt);
    for (int sp = 1; sp < splits; ++sp) {
      f32x4_t v[8];
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) v[tt] = load(sp, i, tt);
#pragma unroll
      for (int tt = 0; tt < 8; ++tt) sum[tt] += v[tt];
    }
#pragma unroll
    for (int tt = 0; tt < 8; ++tt) {
      if (16 * i + l16 < rows_valid) {
        if constexpr (!DENSE) {
#pragma unroll
          for (int v = 0; v < 4; ++v) sum[tt][v] = graded_nonfinite_to_nan(sum[tt][v]);
        }
        out4(i, tt, sum[tt]);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  if (tid == 0) __hip_atomic_store(&p.counters[jt], 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// ------------------------------------------------------------------ x repack

// xt = x in A-fragment order (the layout prefill_tall_kernel reads): 16-row
// tile T, 32-column k step kk -> 1 KiB at (T * K / 32 + kk) KiB, lane l of it
// holding x[16 T + l % 16][32 kk + 8 (l / 16) .. + 7]; rows past M are zero.
// One block per (row tile, 128 columns): each thread reads 16 bytes of one row
// (256 contiguous bytes per row) and writes them where the fragment lane
// that takes them sits.
__global__ __launch_bounds__(256) void repack_x_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M, int K,
                                                       uint16_t* __restrict__ xt) {
  const int T = blockIdx.y, c0 = blockIdx.x * 128;
  const int r = threadIdx.x >> 4, c = threadIdx.x & 15;  // row in tile, 8-column chunk
  const int col = c0 + 8 * c;
  if (col >= K) return;
  const int row = 16 * T + r;
  u32x4_t v = u32x4_t{0u, 0u, 0u, 0u};
  if (row < M) v = *reinterpret_cast<const u32x4_t*>(&x[(int64_t)row * ldx + col]);
  const int kk = col >> 5, lane = r + 16 * ((col >> 3) & 3);
  *reinterpret_cast<u32x4_t*>(&xt[((int64_t)T * (K / 32) + kk) * 512 + lane * 8]) = v;
}

size_t tall_x_bytes(int64_t M, int64_t K) { return (size_t)((M + 15) / 16) * 16 * (size_t)K * 2; }

int launch_repack_x(const uint16_t* x, int64_t ldx, int M, int K, uint16_t* xt, hipStream_t st) {
  if (M <= 0 || K % 32 != 0 || ldx % 8 != 0) return GRINQH_ERR_INVALID;
  const dim3 grid((unsigned)((K + 127) / 128), (unsigned)((M + 15) / 16));
  hipLaunchKernelGGL(repack_x_kernel, grid, dim3(256), 0, st, x, ldx, M, K, xt);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

// ------------------------------------------------------------------ planning

bool prefill_tall_applies(int64_t M, int64_t K, int64_t N, int64_t ldx, int gs) {
  (void)ldx;  // x is repacked first; the repacked copy is addressed with 32-bit offsets
  const bool rows_ok = M >= kTallPrefillRows || (M >= kTallWideRows && (N / 16) / kTallWords >= kTallWideColBlocks);
  return rows_ok && K % kTallBK == 0 && gs % kTallBK == 0 && (N / 16) % kTallWords == 0 &&
         tall_x_bytes(M, K) < ((size_t)1 << 31);
}

// Block height (RT = 8: 512 rows, or 4: 256 rows; one block per CU either
// way) and the split of the last round: the launch should fill the 256 CUs in
// as few rounds of as few stages as possible.  Whole tiles fill full rounds
// (dp_tiles); the tiles left over (or all of them) split K into 2..4 ranges,
// so that the last round is shorter instead of partly empty.  Cost in units
// of one 512-row block's stage: rounds * stages per item * (1 for RT = 8;
// for RT = 4, half the MFMAs and the same dequantization, 0.62 when the
// launch is one round and 0.85 over several), plus the partial sums of the
// split tiles (written by all ranges but one, read once) at about 9 MB per
// unit.  The two RT = 4 factors are fitted to kernel times (MI355X, dense
// fp16): one round, 0.6-0.7 (qkv at 512 rows: 50 us against 60 us for
// 512-row blocks in four K ranges; o_proj at 1024: 55 against 65 us);
// several rounds, 0.85-0.89 (gate_up at 768 rows: 323 us in 256-row blocks
// over 2 rounds and a 3-way split tail, 266 us in 512-row blocks; qkv at
// 2048: 172 against 124 us).
TallPlan plan_tall(int64_t M, int64_t K, int64_t N, size_t max_partial) {
  const int64_t stages = K / kTallBK;
  const int64_t col_blocks = (N / 16) / kTallWords;
  constexpr int64_t slots = 256;
  TallPlan best{8, 1, 0, 0};
  double best_cost = 1e300;
  for (int rt : {8, 4}) {
    const int64_t rows = 64 * rt;
    const int64_t tiles = ((M + rows - 1) / rows) * col_blocks;
    auto f = [rt](int64_t rounds) { return rt == 8 ? 1.0 : rounds <= 1 ? 0.62 : 0.85; };
    auto consider = [&](int s, int64_t dp, double cost) {
      if (cost < best_cost - 1e-9) {
        best_cost = cost;
        best = TallPlan{rt, s, (int)dp, (int)tiles};
      }
    };
    const int64_t rounds_whole = (tiles + slots - 1) / slots;
    consider(1, tiles, (double)rounds_whole * (double)stages * f(rounds_whole));
    for (int64_t dp : {tiles / slots * slots, (int64_t)0}) {
      const int64_t tail = tiles - dp;
      if (tail == 0 || tail > kMaxCounters) continue;
      for (int s = 2; s <= 4; ++s) {
        const size_t part = (size_t)tail * (size_t)s * (size_t)rows * 128 * 4;
        if (stages / s < 8 || part > max_partial) continue;
        const int64_t rounds_dp = dp / slots, rounds_tail = (tail * s + slots - 1) / slots;
        const double traffic = (double)tail * (double)(s - 1) * (double)rows * 128.0 * 4.0 * 2.0 / 9.0e6;
        consider(s, dp,
                 ((double)rounds_dp * (double)stages + (double)rounds_tail * (double)((stages + s - 1) / s)) *
                         f(rounds_dp + rounds_tail) +
                     traffic);
      }
    }
  }
  return best;
}

template <typename DT, int Z, int RT>
static void launch_tall_t(const PrefillParams& p, bool dense, hipStream_t st) {
  constexpr int rows = 64 * RT;
  const int tiles = ((p.M + rows - 1) / rows) * (p.NW / kTallWords);
  const dim3 grid((unsigned)(p.dp_tiles + (tiles - p.dp_tiles) * p.splits));
  if (dense)
    launch_main_kernel(prefill_tall_kernel<DT, Z, true, RT>, grid, dim3(256), st, p);
  else
    launch_main_kernel(prefill_tall_kernel<DT, Z, false, RT>, grid, dim3(256), st, p);
}

template <typename DT, int RT>
static int launch_tall_rt(const PrefillParams& p, int Z, bool dense, hipStream_t st) {
  switch (Z) {
    case 1: launch_tall_t<DT, 1, RT>(p, dense, st); break;
    case 2: launch_tall_t<DT, 2, RT>(p, dense, st); break;
    case 3: launch_tall_t<DT, 3, RT>(p, dense, st); break;
    case 4: launch_tall_t<DT, 4, RT>(p, dense, st); break;
    default: return GRINQH_ERR_INVALID;
  }
  return GRINQH_OK;
}

int launch_prefill_tall(const PrefillParams& p, const TallPlan& plan, int max_bits, int dtype, bool dense,
                        hipStream_t st) {
  if (!dense && p.grades == nullptr) return GRINQH_ERR_INVALID;
  if (!prefill_tall_applies(p.M, p.K, p.N, p.ldx, p.gs) || p.splits != plan.splits || p.splits < 1 ||
      p.dp_tiles != plan.dp_tiles)
    return GRINQH_ERR_INVALID;
  if (plan.rt != 8 && plan.rt != 4) return GRINQH_ERR_INVALID;
  const int64_t rows = 64 * plan.rt;
  const int64_t tiles = ((p.M + rows - 1) / rows) * (p.NW / kTallWords);
  if (plan.tiles != tiles || p.dp_tiles < 0 || p.dp_tiles > tiles || (p.splits == 1) != (p.dp_tiles == tiles) ||
      tiles - p.dp_tiles > kMaxCounters)
    return GRINQH_ERR_INVALID;
  if (p.splits > 1 && (p.partial == nullptr || p.counters == nullptr)) return GRINQH_ERR_INVALID;
  const int Z = max_bits / 2;
  int rc;
  if (dtype == GRINQH_DTYPE_BF16)
    rc = plan.rt == 8 ? launch_tall_rt<BF16, 8>(p, Z, dense, st) : launch_tall_rt<BF16, 4>(p, Z, dense, st);
  else
    rc = plan.rt == 8 ? launch_tall_rt<F16, 8>(p, Z, dense, st) : launch_tall_rt<F16, 4>(p, Z, dense, st);
  if (rc != GRINQH_OK) return rc;
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
