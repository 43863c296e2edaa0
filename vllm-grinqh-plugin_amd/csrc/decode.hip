// Decode-regime GRINQH product (M <= 64 per launch): graded or dense
// y = x * W_eff on v_mfma_f32_16x16x32_{f16,bf16}, HBM-bound.
//
// Replaces the reference's Triton GEMVs grinqh_gemv_uint32_packed
// (grinqh/kernel.py:39-167, one row) and grinqh_gemv_uint32_packed_batch_union
// (:170-360, batch union), and the dense branch of grinqh_gemm_or_gemv for
// small batches (:663-680, semantics of :561-587).
//
// Work decomposition
//   block   = (column block, K range), one-dimensional grid renumbered per XCD
//   column block: 16 plane-word columns w0..w0+15 = 256 logical columns (16
//             column tiles r of 16 contiguous columns r*NW + w0 + c); two
//             neighbours share every 128-byte line of the planes
//   K range = `tiles_per_split` 32-row tiles (split-K)
//   waves   = groups of output dwords j x K sub-ranges: 8 waves (two per
//             SIMD) as 2 dword pairs x 4 sub-ranges for 5-16 rows and for
//             17-64 rows in fp16; 4 waves as MT dword groups x 4/MT
//             sub-ranges for 17-64 rows in bf16
//
// Phase 1 (whole block): stage the scales (and, up to 16 rows, x[:, K range])
// in LDS, grade every row (sigma = max_m |x|, zone bits, midpoint bias) and
// precompute each (row, plane) byte offset, with bit 31 set for planes the
// row does not need.
//
// Phase 2 (per wave): for each tile, each lane (c = lane&15, q = lane>>4) loads
// one 32-bit plane word per (row, plane) of its 8 rows with raw buffer loads;
// offsets with bit 31 set fall past the buffer end and return 0 without a
// memory access, so only the planes a row needs are fetched and no load is
// branched around.  One or two tiles of loads stay in flight while the
// current tile is unpacked.  Code bytes are rebuilt branch-free:
// G_z = rot(D_z, 2z), H_j = field merge of the G_z, V_j = rot(H_j, -2j); then
// turned into the MFMA B operand in one of two ways:
//   - code bytes (5-16 rows, and bf16): fp16 B = u as the subnormal u*2^-24
//     (one v_perm per register), bf16 B = u; the offset 128 and the midpoint
//     bias beta are removed by one extra MFMA per tile whose B operand is the
//     per-row value beta*2^sh - 128 (a "correction column" shared by all 16
//     columns), and per scale group y += s[g][n] * 2^-sh * (C[m][n] + Cv[m])
//     in fp32, as grinqh/kernel.py:148-158 applies scales;
//   - the scaled weight (17-64 rows in fp16): B = RNE(w_eff * s) in fp16,
//     accumulated straight into y (no per-group sums, no correction column).
// Above 16 rows the A operand (x) is not staged for the whole K range: in
// fp16 the two waves that share a K sub-range each load half of the next
// tile's x straight into LDS (buffer loads to LDS) and read the whole tile
// from there, after a per-tile handshake through LDS flags, so each x tile is
// fetched once per K sub-range instead of once per wave; bf16 loads it from
// L2 with the tile's plane words.
//
// Split-K partials are reduced deterministically: the K sub-ranges of a block
// through LDS in fixed order; the K ranges of the grid either by the range
// that finishes last (small reductions: in range order) or by a second kernel
// (in strided lane sums joined by a fixed butterfly), both in fp32 before the
// output cast and bias, in an order that does not depend on timing.
#include "grinqh_common.h"
#include "grinqh_launch.h"
#include "splitk_complete.h"

namespace grinqh {

constexpr int kDecodeRowsPerBlock = 2048;  // rows per block at MT = 1 (x staged in LDS)

// 17-64 rows in fp16 ("scaled" path) multiply the scaled weight RNE(w * s),
// built in registers as the prefill builds it in LDS, and accumulate the
// output directly: no per-group partial sums, no correction column, no group
// epilogue.  The registers this frees let a wave cover two output dwords of all
// 64 rows (128 sums per lane), so the eight waves are two output-dword pairs x
// four K sub-ranges: each plane word and x element is loaded and unpacked by
// two waves (one per dword pair) instead of four.  The weight is rounded once to fp16, as in the
// reference's dense path (grinqh/kernel.py:586).
template <typename DT, int MT>
constexpr bool decode_scaled() { return MT >= 2 && DT::id == F16::id; }
template <typename DT, int MT>
constexpr int decode_waves() { return (decode_scaled<DT, MT>() || MT == 1) ? 8 : 4; }

template <typename DT, int MT, int Z, bool DENSE>
__global__ __launch_bounds__((64 * decode_waves<DT, MT>()), 1) void decode_kernel(DecodeParams p) {
  constexpr bool SC = decode_scaled<DT, MT>();
  constexpr int NWV = decode_waves<DT, MT>();
  constexpr int NT = 64 * NWV;         // threads per block
  constexpr int MP = 16 * MT;          // padded rows of x
  constexpr int NJ = NWV == 8 ? 2 : 4 / MT;  // output dwords j per wave
  constexpr int KW = NWV == 8 ? 4 : 4 / MT;  // K sub-ranges per block
  constexpr int JG = NWV / KW;         // groups of output dwords (waves per K sub-range)
  // tiles of loads in flight ahead of the one unpacked; the scaled path runs
  // two waves per SIMD on 256 registers, with one tile ahead (33-64 rows) or
  // two (17-32 rows), and its A operand through LDS
  constexpr int PF = (SC && MT == 4) ? 1 : 2;
  // 17-64 rows in fp16: the JG waves of a K sub-range share its x tiles
  // through LDS (see s_xr0), each loading XF of a tile's MT fragments.  bf16
  // (one wave per SIMD, none to cover a wave's wait at the handshake) loads
  // them with the plane words two tiles ahead: shared, its 48-64-row
  // products took 17-25 % longer.
  constexpr bool XL = SC;
  constexpr int XF = MT / JG;
  static_assert(!XL || (XF >= 1 && XF * JG == MT), "each wave of a K sub-range loads whole fragments");
  constexpr int SH = 8 - 2 * Z;
  // Up to 16 rows x is staged in LDS for the block's K range; above that the
  // A operand comes tile by tile from global memory (L2-resident; through the
  // shared LDS slots in fp16, with the plane words in bf16), and grading
  // uses the batch statistic of the block's rows, reduced from x
  // in the prologue (or given by the caller), so the K range is not limited
  // by staging x.
  constexpr bool AG = MT >= 2;
  constexpr int RMAX = AG ? kDecodeRowsPerBlock : kDecodeRowsPerBlock / MT;
  static_assert(!AG || RMAX / 8 <= 64 * decode_waves<DT, MT>(), "one statistic chunk per thread");
  constexpr int XS = RMAX + 8;  // halves per staged x row (16-byte rows, banks staggered)
  constexpr int X_BYTES = AG ? 0 : MP * XS * 2;
  constexpr int OFF_BYTES = RMAX * Z * 4;
  // f32x4 slots for the in-block reduction, done one m-tile at a time
  constexpr int RED_VECS = (KW - 1) * JG * NJ * 4 * 64;
  constexpr int POOL_BYTES = (X_BYTES + OFF_BYTES) > RED_VECS * 16 ? (X_BYTES + OFF_BYTES) : RED_VECS * 16;
  constexpr int SC_GROUPS = RMAX / 32 + 1;  // scale groups a K range can touch (group size >= 32)
  constexpr int CPR = RMAX / 8;             // 16-byte x chunks per staged row
  constexpr int XPT = AG ? 1 : MP * CPR / NT;  // x chunks per thread
  constexpr int SPT = (SC_GROUPS * 32 + NT - 1) / NT;  // 16-byte scale chunks per thread

  // staging area: x rows and (row, plane) offsets; reused for the in-block reduction
  __shared__ __align__(16) unsigned char s_pool[POOL_BYTES];
  __shared__ __align__(16) uint16_t s_bv[RMAX];    // row -> correction-column value
  __shared__ __align__(16) uint32_t s_xm[RMAX];    // row -> zone-0 flip
  __shared__ __align__(16) uint16_t s_scale[SC_GROUPS * 256];  // (group, tile, column) scales
  __shared__ uint32_t s_smax;  // graded scaled path: largest |scale| (fp16 bits) above the overflow limit
  // above 16 rows, graded, no statistic given: this block's rows of the batch
  // statistic, max_m |x[m][k]| as float bits (an entry that is NaN in every
  // row gives 0; every output of such a batch is NaN whatever its grading)
  // 17-64 rows in fp16: the x tile of each K sub-range (the A operand of its
  // JG waves) comes into LDS by direct buffer-to-LDS loads one tile ahead,
  // each wave loading XF of its fragments, in PF + 1 slots (one per tile buffer of
  // the unrolled loop) that are separate LDS arrays (so that the compiler's
  // wait for one slot's loads does not also wait for the others').
  // s_xflag[w] is the last tile whose half wave w has in LDS.  The statistic
  // above shares the first slot's storage: it is read only before the first
  // of those loads.
  constexpr int XR_BYTES = XL ? KW * MT * 1024 : 0;
  constexpr int SIG_BYTES = AG ? RMAX * 4 : 4;
  __shared__ __align__(16) unsigned char s_xr0[XR_BYTES > SIG_BYTES ? XR_BYTES : SIG_BYTES];
  __shared__ __align__(16) unsigned char s_xr1[XR_BYTES > 16 ? XR_BYTES : 16];
  __shared__ __align__(16) unsigned char s_xr2[(XL && PF == 2 && XR_BYTES > 16) ? XR_BYTES : 16];
  __shared__ int s_xflag[NWV];
  uint32_t* s_sig = reinterpret_cast<uint32_t*>(s_xr0);
  uint16_t* s_x = reinterpret_cast<uint16_t*>(s_pool);
  uint32_t* s_off = reinterpret_cast<uint32_t*>(s_pool + X_BYTES);
  f32x4_t* s_red = reinterpret_cast<f32x4_t*>(s_pool);

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int jg = wave % JG, kw = wave / JG;
  if (XL && lane == 0) s_xflag[wave] = -(1 << 30);  // read by the partner only after the next barrier
  const int c = lane & 15, q = lane >> 4;
  // logical block = (column block, K range), column blocks fastest, ranges of
  // consecutive logical blocks per XCD (adjacent column blocks share lines)
  const int col_blocks = (p.NW + 15) >> 4;
  const int lb = xcd_chunked(blockIdx.x, gridDim.x);
  const int w0 = (lb % col_blocks) * 16;
  const int split = lb / col_blocks;
  const int ntiles_total = p.K >> 5;
  const int tile0 = split * p.tiles_per_split;
  const int tile1 = min(tile0 + p.tiles_per_split, ntiles_total);
  const int nt = tile1 - tile0;
  const int R = nt * 32;
  const int row0 = tile0 * 32;
  const int g_first = row0 / p.gs;
  const int n_groups = (row0 + R - 1) / p.gs - g_first + 1;

  // Graded scaled path: RNE(w * s) overflows fp16 where |w| * |s| > 65504
  // (|w| <= 2^(2Z-1)), which the reference's fp32 products do not.  A block
  // whose scales reach past kScaleLimit multiplies them by 2^-e in LDS and its
  // sums by 2^e (both exact, except for scales that become subnormal).
  constexpr bool GUARD = SC && !DENSE;
  constexpr uint32_t kScaleLimit = 0x7BFFu - ((uint32_t)(2 * Z - 1) << 10);  // 65504 / 2^(2Z-1), fp16 bits
  uint32_t smax = 0;  // largest |scale| bits this thread staged
  if (GUARD && threadIdx.x == 0) s_smax = 0;
  const bool own_sigma = AG && !DENSE && p.sigma == nullptr;  // block-uniform
  if (own_sigma)
    for (int i = tid; i < R; i += NT) s_sig[i] = 0u;

  float sig_part[8];  // this thread's maxima of K chunk sig_chunk (-1: none)
  int sig_chunk = -1;

  // ---- phase 1a: stage x[:, row0 .. row0+R) in LDS (up to 16 rows) or reduce
  // the block's statistic from it, and load the scales.  The scales are stored
  // to LDS only once the first tiles' plane loads are issued, so their memory
  // round trip overlaps those loads; they are loaded after every x load, so
  // that waiting for x does not wait for them.  Out-of-range buffer offsets
  // read 0: rows m >= M stage as zeros, and nothing past the end of x or the
  // scale array is touched.
  const bool vec_scales = (p.NW % 8) == 0 && (reinterpret_cast<uintptr_t>(p.scale) & 15u) == 0;
  u32x4_t sv[SPT];
  {
    const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.x), (short)0, (int)((uint64_t)p.M * p.ldx * 2u), 0x00020000);
    const uint32_t sbytes = (uint32_t)((uint64_t)((p.K + p.gs - 1) / p.gs) * p.N * 2u);
    const __amdgpu_buffer_rsrc_t sr = __builtin_amdgcn_make_buffer_rsrc(
        const_cast<uint16_t*>(p.scale), (short)0, (int)sbytes, 0x00020000);
    const int u = tid % CPR, mb = tid / CPR;
    u32x4_t xv[XPT];
#pragma unroll
    for (int k = 0; k < XPT; ++k) {
      if constexpr (AG) break;
      const int m = mb + k * (NT / CPR);
      const uint32_t off =
          (m < p.M && 8 * u < R) ? (uint32_t)(((int64_t)m * p.ldx + row0 + 8 * u) * 2) : 0x80000000u;
      xv[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
    }
    if constexpr (!AG) {
#pragma unroll
      for (int k = 0; k < XPT; ++k) {
        const int m = mb + k * (NT / CPR);
        *reinterpret_cast<u32x4_t*>(&s_x[m * XS + 8 * u]) = xv[k];
      }
    }
    // the block's statistic: thread t takes K chunk u0 = t % U (8 rows of K)
    // for batch rows t / U, t / U + S, ... (U = R / 8 <= NT chunks, S = NT / U
    // slices), 8 loads at a time
    if (AG && own_sigma) {
      const int U = R >> 3, S = NT / U;
      const int u0 = tid % U, sl = tid / U;
      if (sl < S) {
        float mx[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) mx[e] = 0.f;
        for (int m0 = sl; m0 < p.M; m0 += 8 * S) {
          u32x4_t v[8];
#pragma unroll
          for (int i = 0; i < 8; ++i) {
            const int m = m0 + i * S;
            const uint32_t off = m < p.M ? (uint32_t)(((int64_t)m * p.ldx + row0 + 8 * u0) * 2) : 0x80000000u;
            v[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
          }
#pragma unroll
          for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              mx[2 * e] = fmaxf(mx[2 * e], fabsf(to_f32<DT>((uint16_t)(v[i][e] & 0xFFFFu))));
              mx[2 * e + 1] = fmaxf(mx[2 * e + 1], fabsf(to_f32<DT>((uint16_t)(v[i][e] >> 16))));
            }
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) sig_part[e] = mx[e];
        sig_chunk = u0;
      }
    }
#pragma unroll
    for (int k = 0; k < SPT; ++k) {
      const int h = tid + NT * k;  // (group, tile, half) chunk
      const int gl = h >> 5, r = (h >> 1) & 15, hf = h & 1;
      const uint32_t off =
          (gl < n_groups && vec_scales)
              ? (uint32_t)(((int64_t)(g_first + gl) * p.N + (int64_t)r * p.NW + w0 + 8 * hf) * 2)
              : 0x80000000u;
      sv[k] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(sr, (int)off, 0, 0));
    }
  }
  __syncthreads();

  if (AG && own_sigma) {
    if (sig_chunk >= 0) {
#pragma unroll
      for (int e = 0; e < 8; ++e)
        if (sig_part[e] > 0.f) atomicMax(&s_sig[8 * sig_chunk + e], __float_as_uint(sig_part[e]));
    }
    __syncthreads();
  }

  // ---- phase 1b: grade each row: correction-column value, zone-0 flip and
  // plane offsets.  Rows with zone 0 active are consumed in offset binary (zone
  // 0's digits flipped, u = int8(U & mask) + 128, and the column value removes
  // the 128); other rows have bit 7 clear and need no flip:
  //   w_eff * 2^sh = u + beta * 2^sh - (zone 0 active ? 128 : 0).
  // A row with no active zone therefore contributes exact zeros.
  // (the loop that reads the caller's statistic from global memory is kept
  // apart, so that the others have no global load and the scale loads stay in
  // flight through them)
  auto grade_row = [&](int rr, float s) {
    uint32_t bits = (1u << Z) - 1u;
    if constexpr (!DENSE) bits = zone_bits<Z>(s, p.thr.t);
    const int beta = DENSE ? 0 : midpoint_bias<Z>(bits);
    if constexpr (SC)  // -c_row of the scaled weight (u >> sh) - c_row, an exact fp16 integer
      s_bv[rr] = f32_to_f16_bits(-(float)(1024 + ((bits & 1u) ? (128 >> SH) : 0) - beta));
    else
      s_bv[rr] = BOperand<DT>::correction(beta * (1 << SH) - ((bits & 1u) ? 128 : 0));
    s_xm[rr] = zone0_flip(bits);
    const uint32_t row_bytes = (uint32_t)(row0 + rr) * (uint32_t)(Z * p.NW) * 4u;
#pragma unroll
    for (int z = 0; z < Z; ++z)
      s_off[rr * Z + z] = ((bits >> z) & 1u) ? row_bytes + (uint32_t)z * (uint32_t)p.NW * 4u : 0x80000000u;
  };
  if (DENSE) {
    for (int rr = tid; rr < R; rr += NT) grade_row(rr, 0.f);
  } else if (AG && own_sigma) {  // this block's share of the batch statistic
    for (int rr = tid; rr < R; rr += NT) grade_row(rr, __uint_as_float(s_sig[rr]));
  } else if (AG || p.sigma != nullptr) {  // the batch statistic given by the caller
    for (int rr = tid; rr < R; rr += NT) grade_row(rr, precomputed_sigma(p, row0 + rr));
  } else {  // from the staged x
    for (int rr = tid; rr < R; rr += NT) {
      float s = fabsf(to_f32<DT>(s_x[rr]));
      for (int m = 1; m < p.M; ++m) s = fmaxf(s, fabsf(to_f32<DT>(s_x[m * XS + rr])));
      grade_row(rr, s);
    }
  }
  __syncthreads();

  int up_exp = 0;  // the block's sums are scaled by 2^up_exp at the end
  // The scales into LDS, once the first tiles' plane loads are issued; then
  // the overflow guard.  The barriers carry no memory fence, so they do not
  // wait for those plane loads, only for the LDS accesses before them.  One
  // staging path per block: where the 16-byte loads were not issued their
  // zero fill would race with the element-wise stores to the same LDS words.
  auto stage_scales = [&]() {
    if (vec_scales) {
#pragma unroll
      for (int k = 0; k < SPT; ++k) {
        const int h = tid + NT * k;
        if ((h >> 5) < SC_GROUPS)
          *reinterpret_cast<u32x4_t*>(&s_scale[(h >> 5) * 256 + ((h >> 1) & 15) * 16 + 8 * (h & 1)]) = sv[k];
        if constexpr (GUARD) {
#pragma unroll
          for (int e = 0; e < 4; ++e) smax = max(smax, max(sv[k][e] & 0x7FFFu, (sv[k][e] >> 16) & 0x7FFFu));
        }
      }
    } else {  // column count not a multiple of 128: element-wise scale staging
      for (int idx = tid; idx < n_groups * 256; idx += NT) {
        const int gl = idx >> 8, col = idx & 255;
        const int wcol = min(w0 + (col & 15), p.NW - 1);
        s_scale[idx] = p.scale[(int64_t)(g_first + gl) * p.N + (int64_t)(col >> 4) * p.NW + wcol];
        if constexpr (GUARD) smax = max(smax, (uint32_t)s_scale[idx] & 0x7FFFu);
      }
    }
    if (GUARD && smax > kScaleLimit) atomicMax(&s_smax, smax);
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    if constexpr (GUARD) {
      const uint32_t hm = s_smax;  // block-uniform
      if (hm > kScaleLimit) {
        up_exp = (int)(hm >> 10) - (int)(kScaleLimit >> 10);
        const float down = __builtin_ldexpf(1.f, -up_exp);
        for (int idx = tid; idx < n_groups * 256; idx += NT)
          s_scale[idx] = from_f32<DT>(to_f32<DT>(s_scale[idx]) * down);
        asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
      }
    }
  };

  // ---- phase 2: main loop over this wave's tiles
  f32x4_t Y[MT][NJ][4];
  f32x4_t C[MT][NJ][4];
  f32x4_t Cv[MT];
#pragma unroll
  for (int mt = 0; mt < MT; ++mt)
#pragma unroll
    for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
      for (int b = 0; b < 4; ++b) Y[mt][jj][b] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  // Lanes past the last word column read the last valid column instead (their
  // outputs are never stored), so every address below is in bounds.
  const bool col_ok = (w0 + c) < p.NW;
  const int wc = col_ok ? (w0 + c) : (p.NW - 1);
  const float post = BOperand<DT>::kUnit / (float)(1 << SH);
  const int t_begin = (nt * kw) / KW, t_end = (nt * (kw + 1)) / KW;
  const int tiles_per_group = p.gs >> 5;

  // Plane words come from raw buffer loads: a (row, plane) a lane does not
  // need has offset bit 31 set, past the buffer end, which returns 0 without a
  // memory access.  The main loop issues every load unconditionally; tiles past
  // the end of the wave's range go through a descriptor of size 0, so every
  // one of their loads returns 0 without touching memory.  Wait counts stay
  // static and two prefetched tiles remain in flight.
  const int plane_bytes = (int)((uint64_t)p.K * (uint32_t)(Z * p.NW) * 4u);
  const __amdgpu_buffer_rsrc_t prsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p.planes), (short)0, plane_bytes, 0x00020000);
  const __amdgpu_buffer_rsrc_t prsrc_none =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(p.planes), (short)0, 0, 0x00020000);
  const uint32_t lane_off = (uint32_t)wc * 4u;

  typedef uint32_t offz_t __attribute__((ext_vector_type(Z)));
  // plane words of one tile (and, above 16 rows, its A operand)
  struct Tile {
    uint32_t D[8][Z];
    u32x4_t A[AG && !XL ? MT : 1];
  };
  const __amdgpu_buffer_rsrc_t xsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.x), (short)0, (int)((uint64_t)p.M * p.ldx * 2u), 0x00020000);
  const __amdgpu_buffer_rsrc_t xsrc_none =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p.x), (short)0, 0, 0x00020000);
  auto issue = [&](int t, Tile& T) {
    const bool live = t < t_end;
    const __amdgpu_buffer_rsrc_t rs = live ? prsrc : prsrc_none;
    const int sb = (live ? t : t_begin) * 32 + 8 * q;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      offz_t o;
      if constexpr (Z == 1) {
        o = s_off[sb + e];
      } else {
        o = *reinterpret_cast<const offz_t*>(&s_off[(sb + e) * Z]);
      }
#pragma unroll
      for (int z = 0; z < Z; ++z) {
        const uint32_t oz = (Z == 1) ? (uint32_t)o[0] : (uint32_t)o[z];
        T.D[e][z] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(rs, (int)(oz + lane_off), 0, 0);
      }
    }
    if constexpr (AG && !XL) {  // x[16*mt + c][rows 8q .. 8q+7 of the tile]; rows m >= M read 0
      const __amdgpu_buffer_rsrc_t xs = live ? xsrc : xsrc_none;
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        const int m = 16 * mt + c;
        const uint32_t off = m < p.M ? (uint32_t)(((int64_t)m * p.ldx + row0 + sb) * 2) : 0x80000000u;
        T.A[mt] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xs, (int)off, 0, 0));
      }
    }
  };

  // one tile: optional prefetch of tile t+2, unpack, MFMA, group epilogue
  // position of the current tile in its scale group and the group's index in
  // the staged scales, advanced per tile (no divisions in the loop)
  int gpos = (tile0 + t_begin) % tiles_per_group;
  int gloc = (tile0 + t_begin) / tiles_per_group - g_first;
  uint32_t s2[NJ][4];  // scaled path: (s, s) of the current group's columns
  // this wave's share of x[16*mt + c][rows 8q .. 8q+7 of tile t] (fragments
  // mt = XF jg .. XF jg + XF - 1) into slot xr: lane l's 16 bytes land at
  // byte 16 l of the fragment's KiB; rows m >= M, and tiles past the range,
  // read nothing (and are never used)
  auto load_x_lds = [&](int t, unsigned char* xr) {
    const __amdgpu_buffer_rsrc_t xs = t < t_end ? xsrc : xsrc_none;
#pragma unroll
    for (int h = 0; h < XF; ++h) {
      const int mt = XF * jg + h;
      const int m = 16 * mt + c;
      const uint32_t off = m < p.M ? (uint32_t)(((int64_t)m * p.ldx + row0 + t * 32 + 8 * q) * 2) : 0x80000000u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(
          xs, (__attribute__((address_space(3))) void*)(xr + (kw * MT + mt) * 1024), 16, (int)off, 0, 0, 0);
    }
  };
  auto step = [&](int t, Tile& Tc, bool prefetch, Tile& Tn, unsigned char* xcur, unsigned char* xnext) {
    const bool first_of_group = (t == t_begin) || (gpos == 0);
    const bool last_of_group = (t + 1 == t_end) || (gpos + 1 == tiles_per_group);
    const int sb = t * 32 + 8 * q;

    // A operand: x[16*mt + c][rows 8q .. 8q+7 of the tile].  At 17-64 rows
    // it is read from the K sub-range's LDS slot, filled in shares by its
    // waves one tile ahead (loaded before the next tile's plane words: memory
    // operations complete in order, so waiting for it leaves those in
    // flight).
    u32x4_t A[MT];
    auto load_a = [&]() {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if constexpr (AG) {
          A[mt] = Tc.A[mt];
        } else {
          A[mt] = *reinterpret_cast<const u32x4_t*>(&s_x[(16 * mt + c) * XS + sb]);
        }
      }
    };
    if constexpr (XL) {
      // own share of tile t (its loads waited for by the compiler), then the
      // handshake: publish it, and wait until every other wave of the K
      // sub-range has published its share, which also means it has read the
      // slots of earlier tiles, the one the next loads overwrite among them.
      // Every wave publishes before it waits, so every wait ends.
      const unsigned char* xb = xcur + kw * MT * 1024 + lane * 16;
      // one dword of the own share read back: the compiler waits for this
      // wave's loads into the slot before it
      const uint32_t probe = *reinterpret_cast<const uint32_t*>(xb + XF * jg * 1024);
      asm volatile("" ::"v"(probe));
      if (lane == 0) __hip_atomic_store(&s_xflag[wave], t, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      // (bounded: a wait that outlasted ~2^20 sleeps would end, with a wrong
      // tile, rather than hang; the others publish within microseconds)
#pragma unroll
      for (int pj = 0; pj < JG; ++pj) {
        if (pj == jg) continue;
        for (int spin = 0; spin < (1 << 20) &&
                           __builtin_amdgcn_readfirstlane(__hip_atomic_load(
                               &s_xflag[kw * JG + pj], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP)) < t;
             ++spin)
          __builtin_amdgcn_s_sleep(1);
      }
      // (always: a tile past the range reads nothing; at 17-32 rows the last
      // two steps take no plane prefetch but the second still needs its x)
      load_x_lds(t + 1, xnext);
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) A[mt] = *reinterpret_cast<const u32x4_t*>(xb + mt * 1024);
    }
    if (prefetch) issue(t + PF, Tn);
    __builtin_amdgcn_sched_barrier(0);
    if constexpr (!XL) load_a();

    const u32x4_t bv = *reinterpret_cast<const u32x4_t*>(&s_bv[sb]);

    // Rebuild the code bytes (offset binary) and turn them into B operands.
    uint32_t xm[8];
    {
      const u32x4_t lo = *reinterpret_cast<const u32x4_t*>(&s_xm[sb]);
      const u32x4_t hi = *reinterpret_cast<const u32x4_t*>(&s_xm[sb + 4]);
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xm[e] = lo[e];
        xm[e + 4] = hi[e];
      }
    }
    prepare_planes<Z>(Tc.D, xm);
    if constexpr (SC) {
      // B = RNE(w * s) with s2 = (s, s) of this lane's columns for the group
      // and bv = (-c_row, -c_row') per row pair; the output accumulates directly.
      if (first_of_group) {
        const uint16_t* srow = &s_scale[gloc * 256 + 64 * jg * NJ + c];
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b) s2[jj][b] = (uint32_t)srow[(4 * jj + b) * 16] * 0x00010001u;
      }
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj) {
        uint32_t V[8];
        code_dwords<Z>(Tc.D, jg * NJ + jj, V);
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          u32x4_t B;
#pragma unroll
          for (int pp = 0; pp < 4; ++pp) B[pp] = Dequant<F16, SH>::pair(V[2 * pp], V[2 * pp + 1], b, bv[pp], s2[jj][b]);
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) Y[mt][jj][b] = mfma16x16x32<DT>(A[mt], B, Y[mt][jj][b]);
        }
      }
    }
#pragma unroll
    for (int jj = 0; jj < (SC ? 0 : NJ); ++jj) {
      const int j = jg * NJ + jj;
      uint32_t V[8];
      code_dwords<Z>(Tc.D, j, V);
      u32x4_t B[4];
      BOperand<DT>::build(V, B);
      // the first tile of a scale group starts its sums from zero
      if (first_of_group) {
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) C[mt][jj][b] = mfma16x16x32<DT>(A[mt], B[b], f32x4_t{0.f, 0.f, 0.f, 0.f});
      } else {
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int mt = 0; mt < MT; ++mt) C[mt][jj][b] = mfma16x16x32<DT>(A[mt], B[b], C[mt][jj][b]);
      }
    }
#pragma unroll
    for (int mt = 0; mt < (SC ? 0 : MT); ++mt)
      Cv[mt] = mfma16x16x32<DT>(A[mt], bv, first_of_group ? f32x4_t{0.f, 0.f, 0.f, 0.f} : Cv[mt]);

    if (!SC && last_of_group) {  // y += s[g][n] * 2^-sh * (C + Cv), scales from LDS
      const uint16_t* srow = &s_scale[gloc * 256 + 64 * jg * NJ + c];
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const float sc = to_f32<DT>(srow[(4 * jj + b) * 16]) * post;
#pragma unroll
          for (int mt = 0; mt < MT; ++mt)
#pragma unroll
            for (int e = 0; e < 4; ++e) Y[mt][jj][b][e] = fmaf(sc, C[mt][jj][b][e] + Cv[mt][e], Y[mt][jj][b][e]);
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
    Tile TA, TB, TC;
    int t = t_begin;
    if constexpr (PF == 2) {
      // three tile buffers: tiles t+1 and t+2 are in flight while tile t is
      // unpacked; the first x tile before the first plane words, as in every
      // step
      if constexpr (XL) load_x_lds(t_begin, s_xr0);
      issue(t_begin, TA);
      issue(t_begin + 1, TB);
      stage_scales();
      for (; t + 3 <= t_end; t += 3) {
        step(t, TA, true, TC, s_xr0, s_xr1);
        step(t + 1, TB, true, TA, s_xr1, s_xr2);
        step(t + 2, TC, true, TB, s_xr2, s_xr0);
      }
      // at most two tiles left, already loaded into TA and TB
      if (t < t_end) step(t, TA, false, TC, s_xr0, s_xr1);
      if (t + 1 < t_end) step(t + 1, TB, false, TC, s_xr1, s_xr2);
    } else {
      // two tile buffers: tile t+1 is in flight while tile t is unpacked
      // the first x tile before the first plane words, as in every step
      if constexpr (XL) load_x_lds(t_begin, s_xr0);
      issue(t_begin, TA);
      stage_scales();
      for (; t + 2 <= t_end; t += 2) {
        step(t, TA, true, TB, s_xr0, s_xr1);
        step(t + 1, TB, true, TA, s_xr1, s_xr0);
      }
      if (t < t_end) step(t, TA, false, TB, s_xr0, s_xr1);
    }
  }

  if (GUARD && up_exp > 0) {
    const float up = __builtin_ldexpf(1.f, up_exp);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt)
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b) Y[mt][jj][b] *= up;
  }

  // ---- phase 3: reduce the K sub-ranges of this block, one m-tile per round.
  // The sums of m-tile mt are added by the waves of K sub-range mt % KW (its
  // owner), in fixed order kw = 0, 1, ..., KW-1, and those waves write that
  // m-tile's outputs, so that the block's stores are spread over its waves:
  // at 64 rows each wave stores 32 values per lane instead of two waves
  // storing 128, which is more agent-scope stores than one wave keeps in
  // flight (it then waits for them to reach memory).  The other sub-ranges
  // leave their sums in the staging area, free now, one slot per wave.
  auto owns = [&](int mt) { return kw == mt % KW; };  // wave-uniform
  if (KW > 1) {
    constexpr int SLOT = NJ * 4 * 64;  // f32x4 per wave slot
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      const int own = mt % KW;
      __syncthreads();
      if (kw != own) {
        f32x4_t* slot = s_red + ((kw < own ? kw : kw - 1) * JG + jg) * SLOT;
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b) slot[(jj * 4 + b) * 64 + lane] = Y[mt][jj][b];
      }
      __syncthreads();
      if (kw == own) {
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b) {
            auto part = [&](int k2) -> f32x4_t {  // sub-range k2's sums
              if (k2 == own) return Y[mt][jj][b];
              return s_red[((k2 < own ? k2 : k2 - 1) * JG + jg) * SLOT + (jj * 4 + b) * 64 + lane];
            };
            f32x4_t acc = part(0);
#pragma unroll
            for (int k2 = 1; k2 < KW; ++k2) acc += part(k2);
            Y[mt][jj][b] = acc;
          }
      }
    }
  }

  // the scaled path multiplies w_eff * s directly: graded rows with a
  // non-finite activation become NaN, as in the reference
  if constexpr (SC && !DENSE) {
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (!owns(mt)) continue;
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int e = 0; e < 4; ++e) Y[mt][jj][b][e] = graded_nonfinite_to_nan(Y[mt][jj][b][e]);
    }
  }

  // ---- phase 4: output (direct, or split-K partials + last-block reduction)
  // Output (m, n) of this lane: m = 16*mt + 4*q + e, n = (4*(jg*NJ+jj)+b)*NW + w0 + c.
  auto col_of = [&](int jj, int b) -> int64_t { return (int64_t)(4 * (jg * NJ + jj) + b) * p.NW + wc; };
  if (p.splits == 1) {
    if (col_ok) {
#pragma unroll
      for (int mt = 0; mt < MT; ++mt) {
        if (!owns(mt)) continue;
#pragma unroll
        for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
          for (int b = 0; b < 4; ++b)
#pragma unroll
            for (int e = 0; e < 4; ++e) {
              const int m = 16 * mt + 4 * q + e;
              if (m < p.M) p.y[(int64_t)m * p.N + col_of(jj, b)] = finish_output<DT>(Y[mt][jj][b][e], p.bias,
                                                                                  (int)col_of(jj, b));
            }
      }
    }
    return;
  }

  // Split-K: this K range's partial sums go to partial[split][m][n]; the
  // range that finishes last (or the reduce kernel that follows on the
  // stream) adds the ranges in fixed order.  Agent-scope (sc1) stores: the
  // last range may read them from another XCD, and before the reduce kernel
  // they stream out during the kernel instead of being written back from L2
  // at its end.  With a slab of partial sums below 2 GiB they are raw buffer
  // stores without branches: the row part of an offset (past the slab for
  // rows m >= M and lanes past the last word column, whose stores the range
  // check drops) in the vector offset, the column tile's part in the scalar
  // offset.
  if ((int64_t)p.M * p.N * 4 < ((int64_t)1 << 31)) {
    const __amdgpu_buffer_rsrc_t prs =
        __builtin_amdgcn_make_buffer_rsrc(p.partial + (int64_t)split * p.M * p.N, (short)0,
                                          (int)((uint32_t)p.M * (uint32_t)p.N * 4u), 0x00020000);
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (!owns(mt)) continue;
      uint32_t roff[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int m = 16 * mt + 4 * q + e;
        roff[e] = (m < p.M && col_ok) ? ((uint32_t)m * (uint32_t)p.N + (uint32_t)wc) * 4u : 0x80000000u;
      }
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b) {
          const uint32_t coff = (uint32_t)(4 * (jg * NJ + jj) + b) * (uint32_t)p.NW * 4u;  // wave-uniform
#pragma unroll
          for (int e = 0; e < 4; ++e)
            __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(Y[mt][jj][b][e]), prs, (int)roff[e], (int)coff,
                                                  kCpolSc1);
        }
    }
  } else if (col_ok) {
    float* part = p.partial + (int64_t)split * p.M * p.N;
#pragma unroll
    for (int mt = 0; mt < MT; ++mt) {
      if (!owns(mt)) continue;
#pragma unroll
      for (int jj = 0; jj < NJ; ++jj)
#pragma unroll
        for (int b = 0; b < 4; ++b)
#pragma unroll
          for (int e = 0; e < 4; ++e) {
            const int m = 16 * mt + 4 * q + e;
            if (m < p.M) store_partial(&part[(int64_t)m * p.N + col_of(jj, b)], Y[mt][jj][b][e]);
          }
    }
  }
  if (p.counters != nullptr) splitk_complete<DT, 4 * MT * 256 / NT, NT>(p, lb % col_blocks, w0, 16);
}

// y[m][n] = cast(sum_{s=0..splits-1} partial[s][m][n]) (+ bias), four
// consecutive columns per chunk.  TPC lanes of one wave share a chunk: lane
// `sub` adds ranges sub, sub + TPC, ... in increasing order (all its loads in
// flight at once), then the TPC sums are combined by a fixed butterfly, so the
// result is the same on every run.
template <typename DT, int TPC>
__global__ __launch_bounds__(256) void splitk_reduce_kernel(const float* __restrict__ partial, int splits, int M,
                                                            int N, const uint16_t* __restrict__ bias,
                                                            uint16_t* __restrict__ y) {
  constexpr int BATCH = 16;
  const int64_t g = (int64_t)blockIdx.x * 256 + threadIdx.x;
  const int64_t i = g / TPC;  // 4-column chunk
  const int sub = (int)(g % TPC);
  const int64_t total = (int64_t)M * N / 4;
  const bool live = i < total;
  const f32x4_t* src = reinterpret_cast<const f32x4_t*>(partial) + (live ? i : 0);
  f32x4_t acc = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int s0 = sub; s0 < splits; s0 += TPC * BATCH) {
    f32x4_t v[BATCH];
#pragma unroll
    for (int k = 0; k < BATCH; ++k) {
      const int s = s0 + k * TPC;
      v[k] = (live && s < splits) ? __builtin_nontemporal_load(src + (int64_t)s * total) : f32x4_t{0.f, 0.f, 0.f, 0.f};
    }
#pragma unroll
    for (int k = 0; k < BATCH; ++k) acc += v[k];
  }
#pragma unroll
  for (int o = TPC / 2; o >= 1; o >>= 1)
#pragma unroll
    for (int e = 0; e < 4; ++e) acc[e] += __shfl_xor(acc[e], o, 64);
  if (!live || sub != 0) return;
  const int n = (int)((i * 4) % N);
  uint16_t o[4];
#pragma unroll
  for (int e = 0; e < 4; ++e) o[e] = finish_output<DT>(acc[e], bias, n + e);
  *reinterpret_cast<u32x2_t*>(y + i * 4) = u32x2_t{(uint32_t)o[0] | ((uint32_t)o[1] << 16),
                                                   (uint32_t)o[2] | ((uint32_t)o[3] << 16)};
}

// sigma_k = max_m |x[m][k]| over the whole batch (NaN ignored unless all NaN,
// as fmaxf does), computed once for kernels that grade from it.  A block
// covers 32 columns; its 8 row groups take every 8th row with 8 loads in
// flight each, and the 8 partial maxima are combined through LDS.  GZ = 0
// writes sigma; GZ = Z writes each row's grade word (grade_word) instead.
template <typename DT, int GZ>
__global__ __launch_bounds__(256) void sigma_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M, int K,
                                                    float* __restrict__ sigma, uint32_t* __restrict__ grades,
                                                    GradeThresholds thr) {
  constexpr int COLS = 32, GROUPS = 256 / COLS, BATCH = 8;
  __shared__ float s_part[GROUPS][COLS];
  const int kk = threadIdx.x % COLS, mg = threadIdx.x / COLS;
  const int k = blockIdx.x * COLS + kk;
  const int kc = min(k, K - 1);  // columns past the end read a valid one and are not stored
  float s = __int_as_float(0x7fc00000);  // NaN: no row seen yet
  for (int m0 = mg; m0 < M; m0 += GROUPS * BATCH) {
    uint16_t v[BATCH];
#pragma unroll
    for (int i = 0; i < BATCH; ++i) {
      const int m = min(m0 + GROUPS * i, M - 1);  // rows past the end repeat the last row
      v[i] = x[(int64_t)m * ldx + kc];
    }
#pragma unroll
    for (int i = 0; i < BATCH; ++i) s = fmaxf(s, fabsf(to_f32<DT>(v[i])));
  }
  s_part[mg][kk] = s;
  __syncthreads();
  if (mg == 0 && k < K) {
#pragma unroll
    for (int g = 1; g < GROUPS; ++g) s = fmaxf(s, s_part[g][kk]);
    if constexpr (GZ == 0)
      sigma[k] = s;
    else
      grades[k] = grade_word<DT, GZ>(s, thr.t);
  }
}

DecodePlan plan_decode(int64_t M, int64_t K, int64_t N) {
  DecodePlan pl{};
  pl.mt = M <= 16 ? 1 : (M <= 32 ? 2 : 4);
  const int64_t NW = N / 16;
  pl.col_blocks = (int)((NW + 15) / 16);
  const int64_t T = K / 32;
  const int kw = pl.mt == 4 ? 4 : 4 / pl.mt;  // K sub-ranges per block (four on the scaled path)
  const int64_t tiles_max = (pl.mt >= 2 ? kDecodeRowsPerBlock : kDecodeRowsPerBlock / pl.mt) / 32;
  const int64_t min_splits = (T + tiles_max - 1) / tiles_max;
  // one block per CU, all blocks resident at once: the per-block set-up
  // (staging, grading) is paid once per CU rather than once per round
  const int64_t want = kTargetBlocks / pl.col_blocks > 0 ? kTargetBlocks / pl.col_blocks : 1;
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
  pl.workspace = splits > 1 ? (size_t)(splits * bytes_per_split) : 0;
  return pl;
}

template <typename DT, int MT, int Z>
static void launch_decode_t(const DecodeParams& p, const DecodePlan& pl, bool dense, hipStream_t st) {
  const dim3 grid(pl.col_blocks * pl.splits);
  const dim3 block(64 * decode_waves<DT, MT>());
  if (dense)
    launch_main_kernel(decode_kernel<DT, MT, Z, true>, grid, block, st, p);
  else
    launch_main_kernel(decode_kernel<DT, MT, Z, false>, grid, block, st, p);
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

template <typename DT, int TPC>
static void launch_reduce_t(const DecodeParams& p, int splits, hipStream_t st) {
  const int64_t chunks = (int64_t)p.M * p.N / 4;
  const dim3 grid((unsigned)((chunks * TPC + 255) / 256));
  hipLaunchKernelGGL((splitk_reduce_kernel<DT, TPC>), grid, dim3(256), 0, st, p.partial, splits, p.M, p.N, p.bias,
                     p.y);
}

template <typename DT>
static void launch_reduce_dt(const DecodeParams& p, int splits, hipStream_t st) {
  // lanes per 4-column chunk: one lane adds up to 16 ranges with all its
  // loads in flight (qkv, o_proj and down at 16 and 64 rows: 3-6 % faster
  // products than four lanes and a butterfly); 64 ranges and more take 16
  // lanes (four lanes of 16 loads each were 5-14 % slower there)
  if (splits >= 64)
    launch_reduce_t<DT, 16>(p, splits, st);
  else if (splits > 16)
    launch_reduce_t<DT, 4>(p, splits, st);
  else
    launch_reduce_t<DT, 1>(p, splits, st);
}

int launch_splitk_reduce(const DecodeParams& p, int splits, int dtype, hipStream_t st) {
  if (dtype == GRINQH_DTYPE_BF16)
    launch_reduce_dt<BF16>(p, splits, st);
  else
    launch_reduce_dt<F16>(p, splits, st);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_sigma(const uint16_t* x, int64_t ldx, int M, int K, int dtype, float* sigma, hipStream_t st) {
  if (K == 0) return GRINQH_OK;
  const dim3 grid((K + 31) / 32);
  const GradeThresholds none{};
  if (dtype == GRINQH_DTYPE_BF16)
    hipLaunchKernelGGL((sigma_kernel<BF16, 0>), grid, dim3(256), 0, st, x, ldx, M, K, sigma, nullptr, none);
  else
    hipLaunchKernelGGL((sigma_kernel<F16, 0>), grid, dim3(256), 0, st, x, ldx, M, K, sigma, nullptr, none);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

template <typename DT>
static void launch_grade_words_dt(const uint16_t* x, int64_t ldx, int M, int K, int Z, const GradeThresholds& thr,
                                  uint32_t* grades, hipStream_t st) {
  const dim3 grid((K + 31) / 32);
  switch (Z) {
    case 1: hipLaunchKernelGGL((sigma_kernel<DT, 1>), grid, dim3(256), 0, st, x, ldx, M, K, nullptr, grades, thr); break;
    case 2: hipLaunchKernelGGL((sigma_kernel<DT, 2>), grid, dim3(256), 0, st, x, ldx, M, K, nullptr, grades, thr); break;
    case 3: hipLaunchKernelGGL((sigma_kernel<DT, 3>), grid, dim3(256), 0, st, x, ldx, M, K, nullptr, grades, thr); break;
    default: hipLaunchKernelGGL((sigma_kernel<DT, 4>), grid, dim3(256), 0, st, x, ldx, M, K, nullptr, grades, thr); break;
  }
}

int launch_grade_words(const uint16_t* x, int64_t ldx, int M, int K, int dtype, int max_bits,
                       const GradeThresholds& thr, uint32_t* grades, hipStream_t st) {
  if (K == 0) return GRINQH_OK;
  if (max_bits < 2 || max_bits > 8 || (max_bits & 1)) return GRINQH_ERR_INVALID;
  if (dtype == GRINQH_DTYPE_BF16)
    launch_grade_words_dt<BF16>(x, ldx, M, K, max_bits / 2, thr, grades, st);
  else
    launch_grade_words_dt<F16>(x, ldx, M, K, max_bits / 2, thr, grades, st);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
