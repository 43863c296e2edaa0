// Dense weight of a large prefill: Wt[n][k] = RNE(w[k][n] * s[k/gs][n]) in the
// activation dtype, stored K-contiguous ([N][K]), for the library GEMM that
// follows (blas.hip).
//
// Replaces the dequantization half of grinqh_prefill_gemm_compiled
// (grinqh/kernel.py:579-586: unpack_pyt + postshuffle + W * s, three torch
// launches over int8 / fp16 copies of the weight).  The values are the same
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
  uint16_t* wt;  // [N][K]
  int K, N, NW, gs;
};

constexpr int kDqColsPerBlock = 32;  // plane-word columns per block (4 waves x 8)
constexpr int kDqRowsPerBlock = 64;  // rows of K per block

template <typename DT, int Z>
__global__ __launch_bounds__(256) void dequant_nk_kernel(DequantParams p) {
  constexpr int SH = 8 - 2 * Z;
  constexpr int LROW = 64 * Z + 4;  // words per word column in LDS (16-byte aligned rows)
  __shared__ __align__(16) uint32_t lds[32 * LROW];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int cb0 = blockIdx.x * kDqColsPerBlock, kb = blockIdx.y * kDqRowsPerBlock;
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

#pragma unroll
  for (int e = 0; e < 8; ++e) {
    D[e][0] ^= 0xAAAAAAAAu;  // offset binary: u = int8(U) + 128
#pragma unroll
    for (int z = 1; z < Z; ++z) D[e][z] = rotr(D[e][z], (uint32_t)(2 * z));
  }
  // every zone active: beta = 0, u - c_row = w * 2^SH
  const uint16_t nc = f32_to_f16_bits(-(float)(1024 + (128 >> SH)));
  const uint32_t negc = (uint32_t)nc | ((uint32_t)nc << 16);
  const float cb = 128.f;

  uint16_t* dst = p.wt + (int64_t)c * p.K + k0;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t out[4][4];  // [beta][pair]
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) {
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
          out[b][pp] = Dequant<BF16, SH>::pair_bf16(V[0], V[1], b, cb, cb, sf);
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

template <typename DT>
int launch_dequant_dt(const DequantParams& p, int max_bits, hipStream_t st) {
  const dim3 grid((unsigned)((p.NW + kDqColsPerBlock - 1) / kDqColsPerBlock),
                  (unsigned)((p.K + kDqRowsPerBlock - 1) / kDqRowsPerBlock));
  switch (max_bits) {
    case 2: launch_main_kernel(dequant_nk_kernel<DT, 1>, grid, dim3(256), st, p); break;
    case 4: launch_main_kernel(dequant_nk_kernel<DT, 2>, grid, dim3(256), st, p); break;
    case 6: launch_main_kernel(dequant_nk_kernel<DT, 3>, grid, dim3(256), st, p); break;
    case 8: launch_main_kernel(dequant_nk_kernel<DT, 4>, grid, dim3(256), st, p); break;
    default: return GRINQH_ERR_INVALID;
  }
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace

int launch_dequant_nk(const uint32_t* planes, const uint16_t* scale, uint16_t* wt, int K, int N, int gs,
                      int max_bits, int dtype, hipStream_t st) {
  if (K % 32 != 0 || N % 64 != 0 || gs % 32 != 0 || (int64_t)K * N >= ((int64_t)1 << 40)) return GRINQH_ERR_INVALID;
  DequantParams p{planes, scale, wt, K, N, N / 16, gs};
  return dtype == GRINQH_DTYPE_BF16 ? launch_dequant_dt<BF16>(p, max_bits, st)
                                    : launch_dequant_dt<F16>(p, max_bits, st);
}

}  // namespace grinqh
