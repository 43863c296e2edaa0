// Load-time layout kernels and integer-exact debug exports: plane pack,
// weight preparation, plane unpack, dequantisation, and the grading export.
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

// S4 plane pack of already preshuffled + shifted bytes U[K][N]
// (reference _pack_kernel_uint32 / pack_triton, grinqh/utils.py:100-146).
// One thread per (k, c): reads the 16 bytes U[k, 16c..16c+15] with one 128-bit
// load and writes word c of every plane.
template <int Z>
__global__ __launch_bounds__(256) void pack_planes_kernel(const uint32_t* __restrict__ U,
                                                          uint32_t* __restrict__ out, int K, int NW) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)K * NW) return;
  const int k = (int)(idx / NW), c = (int)(idx % NW);
  const u32x4_t a = *reinterpret_cast<const u32x4_t*>(U + (int64_t)k * NW * 4 + 4 * c);
#pragma unroll
  for (int z = 0; z < Z; ++z) {
    const uint32_t src = 6 - 2 * z;
    uint32_t w = 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) w |= ((a[i] >> src) & 0x03030303u) << (6 - 2 * i);
    out[((int64_t)k * Z + z) * NW + c] = w;
  }
}

// process_weights_after_loading data path in one pass (grinqh/grinqh.py:200-210):
// logical int8 W[K][N] -> preshuffle (utils.py:17-22) -> << (8-b) -> plane pack.
// Thread (k, c) gathers the 16 logical columns (4j+beta)*NW + c.
template <int Z>
__global__ __launch_bounds__(256) void prepare_weight_kernel(const int8_t* __restrict__ W,
                                                             uint32_t* __restrict__ out, int K, int NW) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)K * NW) return;
  const int k = (int)(idx / NW), c = (int)(idx % NW);
  const int8_t* row = W + (int64_t)k * NW * 16;
  constexpr int SH = 8 - 2 * Z;
  uint32_t u[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) u[r] = ((uint32_t)(uint8_t)row[r * NW + c] << SH) & 0xFFu;
#pragma unroll
  for (int z = 0; z < Z; ++z) {
    uint32_t w = 0;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int j = r >> 2, beta = r & 3;
      w |= ((u[r] >> (6 - 2 * z)) & 3u) << (8 * beta + 6 - 2 * j);
    }
    out[((int64_t)k * Z + z) * NW + c] = w;
  }
}

// S5 unpack of selected rows (reference unpack_pyt, grinqh/utils.py:149-177):
// out[i][16c + 4j + beta] = unsigned b-bit code of U[rows[i], 16c+4j+beta].
template <int Z>
__global__ __launch_bounds__(256) void unpack_planes_kernel(const uint32_t* __restrict__ P,
                                                            const int64_t* __restrict__ rows,
                                                            uint32_t* __restrict__ out, int n_rows,
                                                            int NW) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)n_rows * NW) return;
  const int i = (int)(idx / NW), c = (int)(idx % NW);
  const int64_t k = rows[i];
  uint32_t d[Z];
#pragma unroll
  for (int z = 0; z < Z; ++z) d[z] = P[(k * Z + z) * NW + c];
  u32x4_t o;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    uint32_t w = 0;
#pragma unroll
    for (int z = 0; z < Z; ++z) w |= ((d[z] >> (6 - 2 * j)) & 0x03030303u) << (2 * (Z - 1 - z));
    o[j] = w;
  }
  *reinterpret_cast<u32x4_t*>(out + (int64_t)i * NW * 4 + 4 * c) = o;
}

// F1's unpack + sign extension + postshuffle + scale (grinqh/kernel.py:568-586):
// out[k][n] = RNE_dtype(W[k][n] * scale[k/gs][n]) in the logical column order,
// or the int8 W itself when `scale` is null (then `out` is int8).
template <int Z, typename DT>
__global__ __launch_bounds__(256) void dequant_kernel(const uint32_t* __restrict__ P,
                                                      const uint16_t* __restrict__ scale,
                                                      void* __restrict__ out, int K, int NW, int gs) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)K * NW) return;
  const int k = (int)(idx / NW), c = (int)(idx % NW);
  const int N = NW * 16;
  constexpr int SH = 8 - 2 * Z;
  uint32_t d[Z];
#pragma unroll
  for (int z = 0; z < Z; ++z) d[z] = P[((int64_t)k * Z + z) * NW + c];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int j = r >> 2, beta = r & 3;
    uint32_t code = 0;
#pragma unroll
    for (int z = 0; z < Z; ++z) code = (code << 2) | ((d[z] >> (8 * beta + 6 - 2 * j)) & 3u);
    const int w = ((int)(int8_t)(uint8_t)(code << SH)) >> SH;
    const int64_t n = (int64_t)r * NW + c;
    if (scale == nullptr) {
      static_cast<int8_t*>(out)[(int64_t)k * N + n] = (int8_t)w;
    } else {
      const float s = to_f32<DT>(scale[(int64_t)(k / gs) * N + n]);
      static_cast<uint16_t*>(out)[(int64_t)k * N + n] = from_f32<DT>((float)w * s);
    }
  }
}

// Grading export (reference inline grading, grinqh/kernel.py:98-114 for one
// row and :249-289 for the batch union): per weight row k, the zone bits of
// sigma_k = max_m |x[m][k]| (NaN ignored) and the midpoint bias beta_k.
//
// A column whose entries are all NaN: the reference holds the batch in one
// tile of next_power_of_2(M) rows whose rows past M load as 0.0
// (grinqh/kernel.py:196-197, 240-245, 632) and reduces with a NaN-ignoring
// maximum, so the statistic is 0.0 when M is not a power of two (zone z on
// iff 0 > t_z, the `nan_bits` given here) and NaN, no zone, otherwise.  Only
// this export can show the difference: in a product every output of such a
// batch is NaN whatever the grading.
template <int Z, typename DT>
__global__ __launch_bounds__(256) void grade_kernel(const uint16_t* __restrict__ x, int64_t ldx, int M,
                                                    int K, GradeThresholds thr, uint32_t nan_bits,
                                                    uint8_t* __restrict__ bits, int32_t* __restrict__ beta) {
  const int k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= K) return;
  const float s = column_absmax<DT>(x, ldx, M, k);
  const uint32_t b = s == s ? zone_bits<Z>(s, thr.t) : nan_bits & ((1u << Z) - 1u);
  bits[k] = (uint8_t)b;
  if (beta != nullptr) beta[k] = midpoint_bias<Z>(b);
}

// ---------------------------------------------------------------- launchers

#define GRINQH_SWITCH_Z(Zv, ...)                   \
  switch (Zv) {                                    \
    case 1: { constexpr int Z_ = 1; __VA_ARGS__; } break; \
    case 2: { constexpr int Z_ = 2; __VA_ARGS__; } break; \
    case 3: { constexpr int Z_ = 3; __VA_ARGS__; } break; \
    case 4: { constexpr int Z_ = 4; __VA_ARGS__; } break; \
    default: return GRINQH_ERR_INVALID;            \
  }

static inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

int launch_pack_planes(const uint32_t* U, uint32_t* out, int K, int N, int max_bits, hipStream_t st) {
  const int NW = N / 16;
  if ((int64_t)K * NW == 0) return GRINQH_OK;
  GRINQH_SWITCH_Z(max_bits / 2,
    hipLaunchKernelGGL(pack_planes_kernel<Z_>, dim3(blocks_for((int64_t)K * NW)), dim3(256), 0, st, U, out, K, NW));
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_prepare_weight(const int8_t* W, uint32_t* out, int K, int N, int max_bits, hipStream_t st) {
  const int NW = N / 16;
  if ((int64_t)K * NW == 0) return GRINQH_OK;
  GRINQH_SWITCH_Z(max_bits / 2,
    hipLaunchKernelGGL(prepare_weight_kernel<Z_>, dim3(blocks_for((int64_t)K * NW)), dim3(256), 0, st, W, out, K, NW));
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_unpack_planes(const uint32_t* P, const int64_t* rows, uint32_t* out, int n_rows, int N, int Z,
                         hipStream_t st) {
  const int NW = N / 16;
  if ((int64_t)n_rows * NW == 0) return GRINQH_OK;
  GRINQH_SWITCH_Z(Z,
    hipLaunchKernelGGL(unpack_planes_kernel<Z_>, dim3(blocks_for((int64_t)n_rows * NW)), dim3(256), 0, st, P, rows, out, n_rows, NW));
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_dequant(const uint32_t* P, const uint16_t* scale, void* out, int K, int N, int max_bits, int gs,
                   int dtype, hipStream_t st) {
  const int NW = N / 16;
  if ((int64_t)K * NW == 0) return GRINQH_OK;
  const dim3 grid(blocks_for((int64_t)K * NW));
  if (dtype == GRINQH_DTYPE_BF16) {
    GRINQH_SWITCH_Z(max_bits / 2,
      hipLaunchKernelGGL((dequant_kernel<Z_, BF16>), grid, dim3(256), 0, st, P, scale, out, K, NW, gs));
  } else {
    GRINQH_SWITCH_Z(max_bits / 2,
      hipLaunchKernelGGL((dequant_kernel<Z_, F16>), grid, dim3(256), 0, st, P, scale, out, K, NW, gs));
  }
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_grade(const uint16_t* x, int64_t ldx, int M, int K, const float* t, int max_bits, int dtype,
                 uint8_t* bits, int32_t* beta, hipStream_t st) {
  if (K == 0) return GRINQH_OK;
  GradeThresholds thr;
  uint32_t nan_bits = 0;  // zone bits of an all-NaN column: 0 > t_z when M is not a power of two
  for (int i = 0; i < 4; ++i) {
    thr.t[i] = t[i];
    if ((M & (M - 1)) != 0 && 0.f > t[i]) nan_bits |= 1u << i;
  }
  const dim3 grid(blocks_for(K));
  if (dtype == GRINQH_DTYPE_BF16) {
    GRINQH_SWITCH_Z(max_bits / 2,
      hipLaunchKernelGGL((grade_kernel<Z_, BF16>), grid, dim3(256), 0, st, x, ldx, M, K, thr, nan_bits, bits, beta));
  } else {
    GRINQH_SWITCH_Z(max_bits / 2,
      hipLaunchKernelGGL((grade_kernel<Z_, F16>), grid, dim3(256), 0, st, x, ldx, M, K, thr, nan_bits, bits, beta));
  }
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
