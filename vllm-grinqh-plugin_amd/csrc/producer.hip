// Producer fusion: the operations that feed a GRINQH linear in a Llama-style
// block also emit the batch statistic the union grading needs, so the
// product does not read x once more to build it.
//
//   rmsnorm_sigma:  h = x (+ residual_in; h to residual_out), y = RNE(h * rsqrt(mean(h^2) + eps)) * w
//   silu_mul_sigma: y = RNE(silu(g)) * u for gate_up = [g | u]
//
// Both write y and, for every chunk of kSigmaChunkRows rows, the column maxima
// sigma_chunks[chunk][k] = max over the chunk's rows of |y[m][k]| (fmaxf: NaN
// ignored unless every value is NaN, as the products' own statistic does).
// The maximum over the chunks is sigma_k = max_m |y[m][k]|, the statistic of
// grinqh/kernel.py:249; the products take the chunk maxima directly.
//
// Arithmetic follows vLLM's fused_add_rms_norm and SiluAndMul kernels (the
// operations these replace in the model): the residual sum is rounded to the
// activation dtype and its fp32 square enters the variance; the normalised
// value is rounded to the dtype before the weight multiply; silu is computed
// in fp32 and rounded before the multiply by the up half.
#include "grinqh_common.h"
#include "grinqh_launch.h"

namespace grinqh {

constexpr int kProducerCols = 512;  // columns per block

// Block = kSigmaChunkRows rows x 512 columns, 256 threads.  Phase 1: the
// variance of each of its rows over all K (16 threads per row, 16-byte loads;
// every column block of the chunk repeats it, which costs L2 reads only).
// Phase 2: its 512 columns, each thread 8 columns x 4 rows.  Since every
// column block reads whole rows of residual_in, the sum goes to a separate
// residual_out (writing it back in place would race with those reads).
template <typename DT>
__global__ __launch_bounds__(256) void rmsnorm_sigma_kernel(const uint16_t* __restrict__ x, int64_t ldx,
                                                            const uint16_t* __restrict__ residual,
                                                            uint16_t* __restrict__ residual_out,
                                                            const uint16_t* __restrict__ weight, float eps,
                                                            uint16_t* __restrict__ y, float* __restrict__ sigma_chunks,
                                                            int M, int K) {
  constexpr int R = kSigmaChunkRows;
  __shared__ float s_rstd[R];
  __shared__ float s_max[4][kProducerCols];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.y * R;
  const int c0 = blockIdx.x * kProducerCols;

  // phase 1: row tid / 16, columns 8 * (tid % 16) + 128 * i
  {
    const int row = tid >> 4, sub = tid & 15;
    const int m = r0 + row;
    float ss = 0.f;
    if (m < M) {
      for (int k = 8 * sub; k < K; k += 128) {
        const u32x4_t a = *reinterpret_cast<const u32x4_t*>(x + (int64_t)m * ldx + k);
        u32x4_t r = u32x4_t{0u, 0u, 0u, 0u};
        if (residual != nullptr) r = *reinterpret_cast<const u32x4_t*>(residual + (int64_t)m * K + k);
#pragma unroll
        for (int q = 0; q < 4; ++q)
#pragma unroll
          for (int h = 0; h < 2; ++h) {
            float v = to_f32<DT>((uint16_t)(a[q] >> (16 * h)));
            if (residual != nullptr) v = to_f32<DT>(from_f32<DT>(v + to_f32<DT>((uint16_t)(r[q] >> (16 * h)))));
            ss = fmaf(v, v, ss);
          }
      }
    }
#pragma unroll
    for (int o = 8; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 16);
    if (sub == 0) s_rstd[row] = rsqrtf(ss / (float)K + eps);
  }
  __syncthreads();

  // phase 2: columns c0 + 8 * (tid % 64) .. +7, rows tid / 64 + 4 * i
  const int k = c0 + 8 * (tid & 63);
  const int rb = tid >> 6;
  float mx[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) mx[e] = __int_as_float(0x7fc00000);  // NaN: no row seen yet
  if (k < K) {
    const u32x4_t wv = *reinterpret_cast<const u32x4_t*>(weight + k);
#pragma unroll
    for (int i = 0; i < R / 4; ++i) {
      const int row = rb + 4 * i, m = r0 + row;
      if (m >= M) break;
      const u32x4_t a = *reinterpret_cast<const u32x4_t*>(x + (int64_t)m * ldx + k);
      u32x4_t r = u32x4_t{0u, 0u, 0u, 0u};
      if (residual != nullptr) r = *reinterpret_cast<const u32x4_t*>(residual + (int64_t)m * K + k);
      u32x4_t out, hsum;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t o2 = 0, h2 = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          uint16_t hb = (uint16_t)(a[q] >> (16 * h));
          if (residual != nullptr)
            hb = from_f32<DT>(to_f32<DT>(hb) + to_f32<DT>((uint16_t)(r[q] >> (16 * h))));
          const uint16_t nrm = from_f32<DT>(to_f32<DT>(hb) * s_rstd[row]);
          const uint16_t yb = from_f32<DT>(to_f32<DT>(nrm) * to_f32<DT>((uint16_t)(wv[q] >> (16 * h))));
          mx[2 * q + h] = fmaxf(mx[2 * q + h], fabsf(to_f32<DT>(yb)));
          o2 |= (uint32_t)yb << (16 * h);
          h2 |= (uint32_t)hb << (16 * h);
        }
        out[q] = o2;
        hsum[q] = h2;
      }
      *reinterpret_cast<u32x4_t*>(y + (int64_t)m * K + k) = out;
      if (residual != nullptr) *reinterpret_cast<u32x4_t*>(residual_out + (int64_t)m * K + k) = hsum;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_max[rb][8 * (tid & 63) + e] = mx[e];
  __syncthreads();
  for (int cc = tid; cc < kProducerCols; cc += 256) {
    const int kk = c0 + cc;
    if (kk >= K) break;
    const float v = fmaxf(fmaxf(s_max[0][cc], s_max[1][cc]), fmaxf(s_max[2][cc], s_max[3][cc]));
    sigma_chunks[(int64_t)blockIdx.y * K + kk] = v;
  }
}

// Block = kSigmaChunkRows rows x 512 columns of y [M][F]; gate_up rows hold
// [g (F values) | u (F values)], ld elements apart.
template <typename DT>
__global__ __launch_bounds__(256) void silu_mul_sigma_kernel(const uint16_t* __restrict__ gu, int64_t ld,
                                                             uint16_t* __restrict__ y, float* __restrict__ sigma_chunks,
                                                             int M, int F) {
  constexpr int R = kSigmaChunkRows;
  __shared__ float s_max[4][kProducerCols];
  const int tid = threadIdx.x;
  const int r0 = blockIdx.y * R;
  const int k = blockIdx.x * kProducerCols + 8 * (tid & 63);
  const int rb = tid >> 6;
  float mx[8];
#pragma unroll
  for (int e = 0; e < 8; ++e) mx[e] = __int_as_float(0x7fc00000);
  if (k < F) {
#pragma unroll
    for (int i = 0; i < R / 4; ++i) {
      const int m = r0 + rb + 4 * i;
      if (m >= M) break;
      const u32x4_t g = *reinterpret_cast<const u32x4_t*>(gu + (int64_t)m * ld + k);
      const u32x4_t u = *reinterpret_cast<const u32x4_t*>(gu + (int64_t)m * ld + F + k);
      u32x4_t out;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        uint32_t o2 = 0;
#pragma unroll
        for (int h = 0; h < 2; ++h) {
          const float gv = to_f32<DT>((uint16_t)(g[q] >> (16 * h)));
          const uint16_t act = from_f32<DT>(gv / (1.f + expf(-gv)));
          const uint16_t yb = from_f32<DT>(to_f32<DT>(act) * to_f32<DT>((uint16_t)(u[q] >> (16 * h))));
          mx[2 * q + h] = fmaxf(mx[2 * q + h], fabsf(to_f32<DT>(yb)));
          o2 |= (uint32_t)yb << (16 * h);
        }
        out[q] = o2;
      }
      *reinterpret_cast<u32x4_t*>(y + (int64_t)m * F + k) = out;
    }
  }
#pragma unroll
  for (int e = 0; e < 8; ++e) s_max[rb][8 * (tid & 63) + e] = mx[e];
  __syncthreads();
  for (int cc = tid; cc < kProducerCols; cc += 256) {
    const int kk = blockIdx.x * kProducerCols + cc;
    if (kk >= F) break;
    sigma_chunks[(int64_t)blockIdx.y * F + kk] =
        fmaxf(fmaxf(s_max[0][cc], s_max[1][cc]), fmaxf(s_max[2][cc], s_max[3][cc]));
  }
}

int launch_rmsnorm_sigma(const uint16_t* x, int64_t ldx, const uint16_t* residual, uint16_t* residual_out,
                         const uint16_t* weight, float eps, uint16_t* y, float* sigma_chunks, int M, int K, int dtype,
                         hipStream_t st) {
  const dim3 grid((K + kProducerCols - 1) / kProducerCols, (M + kSigmaChunkRows - 1) / kSigmaChunkRows);
  if (dtype == GRINQH_DTYPE_BF16)
    hipLaunchKernelGGL(rmsnorm_sigma_kernel<BF16>, grid, dim3(256), 0, st, x, ldx, residual, residual_out, weight, eps, y,
                       sigma_chunks, M, K);
  else
    hipLaunchKernelGGL(rmsnorm_sigma_kernel<F16>, grid, dim3(256), 0, st, x, ldx, residual, residual_out, weight, eps, y,
                       sigma_chunks, M, K);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

int launch_silu_mul_sigma(const uint16_t* gu, int64_t ld, uint16_t* y, float* sigma_chunks, int M, int F, int dtype,
                          hipStream_t st) {
  const dim3 grid((F + kProducerCols - 1) / kProducerCols, (M + kSigmaChunkRows - 1) / kSigmaChunkRows);
  if (dtype == GRINQH_DTYPE_BF16)
    hipLaunchKernelGGL(silu_mul_sigma_kernel<BF16>, grid, dim3(256), 0, st, gu, ld, y, sigma_chunks, M, F);
  else
    hipLaunchKernelGGL(silu_mul_sigma_kernel<F16>, grid, dim3(256), 0, st, gu, ld, y, sigma_chunks, M, F);
  return hipGetLastError() == hipSuccess ? GRINQH_OK : GRINQH_ERR_HIP;
}

}  // namespace grinqh
