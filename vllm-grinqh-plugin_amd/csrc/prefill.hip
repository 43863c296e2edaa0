// Prefill-regime GRINQH product (M > 64): dequantize-into-LDS GEMM on
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
// x 16 column tiles); 4 waves as 2 x 2, each BM/2 rows x 8 column tiles.
// Per 32-row stage: A (x) and the dequantized B go to the LDS buffer the MFMAs
// are not reading, global loads for the following stage are in flight while
// the current one is multiplied.
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

constexpr int kPrefillKP = 40;  // halves per LDS row of a 32-row stage (32 + 8 pad: conflict-free)

// Two rows (low half = row 0, high half = row 1) of column tile beta from the
// code dwords V0, V1 (offset-binary bytes u): RNE(w * s) with
// w = (u >> sh) - c_row, c_row = 1024 + (128 >> sh) - beta_row.
template <typename DT, int SH>
struct Dequant;

template <int SH>
struct Dequant<F16, SH> {
  // negc: (-c_row0, -c_row1) as fp16; s2: (s, s) as fp16
  __device__ __forceinline__ static uint32_t pair(uint32_t V0, uint32_t V1, int beta, uint32_t negc, uint32_t s2) {
    uint32_t h = perm(V1, V0, 0x0C040C00u + (uint32_t)beta * 0x00010001u);  // (u0, 0, u1, 0)
    if (SH > 0) h >>= SH;  // the low sh bits of each code byte are zero, so halves do not mix
    h |= 0x64006400u;      // 1024 + (u >> sh), exact
    const half2_t w = __builtin_bit_cast(half2_t, h) + __builtin_bit_cast(half2_t, negc);  // exact integers
    return __builtin_bit_cast(uint32_t, w * __builtin_bit_cast(half2_t, s2));                // RNE(w * s)
  }
};

template <int SH>
struct Dequant<BF16, SH> {
  // negc: per row -c_row * 2^sh... carried as two floats in the caller; here
  // w * s = (u - C_row) * (s * 2^-sh) with C_row = 128 - beta_row * 2^sh: exact
  // in fp32, then one rounding to bf16.
  __device__ __forceinline__ static uint32_t pair_bf16(uint32_t V0, uint32_t V1, int beta, float c0, float c1,
                                                       float s_sh) {
    const float a = (float)((V0 >> (8 * beta)) & 0xFFu) - c0;
    const float b = (float)((V1 >> (8 * beta)) & 0xFFu) - c1;
    return (uint32_t)f32_to_bf16_bits(a * s_sh) | ((uint32_t)f32_to_bf16_bits(b * s_sh) << 16);
  }
};

template <typename DT, int BM, int Z, bool DENSE>
__global__ __launch_bounds__(256, 1) void prefill_kernel(PrefillParams p) {
  constexpr int SH = 8 - 2 * Z;
  constexpr int KP = kPrefillKP;
  constexpr int WM = BM / 2;       // rows per wave
  constexpr int MTW = WM / 16;     // 16-row MFMA tiles per wave
  constexpr int A_HALVES = BM * KP;
  constexpr int B_HALVES = 256 * KP;  // (column tile, column) rows of 32 k
  constexpr int AL = BM * 4 / 256;    // 16-byte A chunks per thread per stage

  __shared__ __align__(16) uint16_t s_a[2][A_HALVES];
  __shared__ __align__(16) uint16_t s_b[2][B_HALVES];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int c = lane & 15, q = lane >> 4;
  const int w0 = blockIdx.x * 16;
  const int m0 = blockIdx.y * BM;
  const int nstages = p.K >> 5;

  // A loader: chunk (row, 16-byte piece): 4 threads per row
  const __amdgpu_buffer_rsrc_t xr = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint16_t*>(p.x), (short)0, (int)((uint64_t)p.M * p.ldx * 2u), 0x00020000);
  // B loader: word column wcol, rows 2*rp and 2*rp + 1 of the stage
  const int wcol = tid & 15, rp = tid >> 4;
  const bool col_ok_ld = (w0 + wcol) < p.NW;
  const int wc_ld = col_ok_ld ? (w0 + wcol) : (p.NW - 1);
  const __amdgpu_buffer_rsrc_t prsrc = __builtin_amdgcn_make_buffer_rsrc(
      const_cast<uint32_t*>(p.planes), (short)0, (int)((uint64_t)p.K * (uint32_t)(Z * p.NW) * 4u), 0x00020000);
  const uint32_t plane_row_bytes = (uint32_t)(Z * p.NW) * 4u;

  u32x4_t xa[AL];
  uint32_t D[2][Z];
  float sig[2];
  uint16_t sraw[16];  // scales of the stage's group when it starts a new group
  bool new_group = false;
  auto load_stage = [&](int s) {
    const int k0 = s * 32;
    new_group = (s == 0) || (k0 / p.gs != (k0 - 32) / p.gs);
    if (new_group) {  // this thread's 16 columns: column tile r, word column wc_ld
      const int g = k0 / p.gs;
#pragma unroll
      for (int r = 0; r < 16; ++r) sraw[r] = p.scale[(int64_t)g * p.N + (int64_t)r * p.NW + wc_ld];
    }
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const int h = tid + 256 * i, row = h >> 2, piece = h & 3;
      const int m = m0 + row;
      const uint32_t off = m < p.M ? (uint32_t)(((int64_t)m * p.ldx + k0 + 8 * piece) * 2) : 0x80000000u;
      xa[i] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(xr, (int)off, 0, 0));
    }
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const uint32_t rb = (uint32_t)(k0 + 2 * rp + e) * plane_row_bytes + (uint32_t)wc_ld * 4u;
#pragma unroll
      for (int z = 0; z < Z; ++z)
        D[e][z] = (uint32_t)__builtin_amdgcn_raw_buffer_load_b32(prsrc, (int)(rb + (uint32_t)z * p.NW * 4u), 0, 0);
      if (!DENSE) sig[e] = p.sigma[k0 + 2 * rp + e];
    }
  };

  // scales of this thread's 16 columns for the current group
  uint32_t s2[16];  // fp16: (s, s)
  float sf[16];     // bf16: s * 2^-sh

  auto store_stage = [&](int buf) {
    // A: straight copy
#pragma unroll
    for (int i = 0; i < AL; ++i) {
      const int h = tid + 256 * i, row = h >> 2, piece = h & 3;
      *reinterpret_cast<u32x4_t*>(&s_a[buf][row * KP + 8 * piece]) = xa[i];
    }
    // B: grade (union), rebuild code bytes, dequantize, write (column tile, column)[k]
    uint32_t bits[2];
    int beta[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      bits[e] = DENSE ? ((1u << Z) - 1u) : zone_bits<Z>(sig[e], p.thr.t);
      beta[e] = DENSE ? 0 : midpoint_bias<Z>(bits[e]);
      if (!DENSE) {
#pragma unroll
        for (int z = 0; z < Z; ++z) D[e][z] &= ((bits[e] >> z) & 1u) ? 0xFFFFFFFFu : 0u;
      }
      D[e][0] ^= 0xAAAAAAAAu;  // offset binary: u = int8(U & mask) + 128
#pragma unroll
      for (int z = 1; z < Z; ++z) D[e][z] = rotr(D[e][z], (uint32_t)(2 * z));
    }
    if (new_group) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (DT::id == F16::id)
          s2[r] = (uint32_t)sraw[r] | ((uint32_t)sraw[r] << 16);
        else
          sf[r] = to_f32<DT>(sraw[r]) * (1.0f / (float)(1 << SH));
      }
    }
    uint32_t negc = 0;
    float cb[2] = {0.f, 0.f};
    if constexpr (DT::id == F16::id) {
      const uint16_t c0 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[0]));
      const uint16_t c1 = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta[1]));
      negc = (uint32_t)c0 | ((uint32_t)c1 << 16);
    } else {
      cb[0] = (float)(128 - beta[0] * (1 << SH));
      cb[1] = (float)(128 - beta[1] * (1 << SH));
    }
    uint16_t* bdst = &s_b[buf][wcol * KP + 2 * rp];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      uint32_t V[2];
#pragma unroll
      for (int e = 0; e < 2; ++e) {
        uint32_t h = (Z == 4) ? D[e][3] : (D[e][0] & (0x03030303u << (2 * ((3 - j) & 3))));
#pragma unroll
        for (int z = (Z == 4 ? 0 : 1); z < (Z == 4 ? 3 : Z); ++z)
          h = bfi(0x03030303u << (2 * ((3 - z - j) & 3)), D[e][z], h);
        V[e] = rotr(h, (uint32_t)(32 - 2 * j) & 31u);
      }
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int r = 4 * j + b;
        uint32_t pr;
        if constexpr (DT::id == F16::id) {
          pr = Dequant<F16, SH>::pair(V[0], V[1], b, negc, s2[r]);
        } else {
          pr = Dequant<BF16, SH>::pair_bf16(V[0], V[1], b, cb[0], cb[1], sf[r]);
        }
        *reinterpret_cast<uint32_t*>(bdst + r * 16 * KP) = pr;
      }
    }
  };

  f32x4_t acc[MTW][8];
#pragma unroll
  for (int i = 0; i < MTW; ++i)
#pragma unroll
    for (int r = 0; r < 8; ++r) acc[i][r] = f32x4_t{0.f, 0.f, 0.f, 0.f};

  load_stage(0);
  store_stage(0);
  __syncthreads();
  for (int s = 0; s < nstages; ++s) {
    const int buf = s & 1;
    if (s + 1 < nstages) load_stage(s + 1);
    // B fragments of this wave's 8 column tiles, then the A tiles one by one
    u32x4_t Bf[8];
#pragma unroll
    for (int r = 0; r < 8; ++r)
      Bf[r] = *reinterpret_cast<const u32x4_t*>(&s_b[buf][((8 * wn + r) * 16 + c) * KP + 8 * q]);
#pragma unroll
    for (int i = 0; i < MTW; ++i) {
      const u32x4_t Af = *reinterpret_cast<const u32x4_t*>(&s_a[buf][(wm * WM + 16 * i + c) * KP + 8 * q]);
#pragma unroll
      for (int r = 0; r < 8; ++r) acc[i][r] = mfma16x16x32<DT>(Af, Bf[r], acc[i][r]);
    }
    if (s + 1 < nstages) store_stage(buf ^ 1);
    __syncthreads();
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
        if (m < p.M) p.y[(int64_t)m * p.N + n] = finish_output<DT>(acc[i][r][e], p.bias, (int)n);
      }
    }
}

template <typename DT, int BM, int Z>
static void launch_prefill_t(const PrefillParams& p, bool dense, hipStream_t st) {
  const dim3 grid((p.NW + 15) / 16, (p.M + BM - 1) / BM);
  if (dense)
    hipLaunchKernelGGL((prefill_kernel<DT, BM, Z, true>), grid, dim3(256), 0, st, p);
  else
    hipLaunchKernelGGL((prefill_kernel<DT, BM, Z, false>), grid, dim3(256), 0, st, p);
}

template <typename DT, int BM>
static int launch_prefill_bm(const PrefillParams& p, int Z, bool dense, hipStream_t st) {
  switch (Z) {
    case 1: launch_prefill_t<DT, BM, 1>(p, dense, st); break;
    case 2: launch_prefill_t<DT, BM, 2>(p, dense, st); break;
    case 3: launch_prefill_t<DT, BM, 3>(p, dense, st); break;
    case 4: launch_prefill_t<DT, BM, 4>(p, dense, st); break;
    default: return GRINQH_ERR_INVALID;
  }
  return GRINQH_OK;
}

// 256-row tiles when they still give one block per CU, else 128-row tiles.
int prefill_block_rows(int64_t M, int64_t N) {
  const int64_t col_blocks = (N / 16 + 15) / 16;
  return col_blocks * ((M + 255) / 256) >= kTargetBlocks ? 256 : 128;
}

template <typename DT>
static int launch_prefill_dt(const PrefillParams& p, int Z, bool dense, hipStream_t st) {
  return prefill_block_rows(p.M, p.N) == 256 ? launch_prefill_bm<DT, 256>(p, Z, dense, st)
                                             : launch_prefill_bm<DT, 128>(p, Z, dense, st);
}

int launch_prefill(const PrefillParams& p, int max_bits, int dtype, bool dense, hipStream_t st) {
  if (!dense && p.sigma == nullptr) return GRINQH_ERR_INVALID;
  const int Z = max_bits / 2;
  const int rc = dtype == GRINQH_DTYPE_BF16 ? launch_prefill_dt<BF16>(p, Z, dense, st)
                                            : launch_prefill_dt<F16>(p, Z, dense, st);
  if (rc != GRINQH_OK) return rc;
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
