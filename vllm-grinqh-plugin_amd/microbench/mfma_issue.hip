// MFMA issue microbenchmark: how many independent VALU instructions one wave
// (or two waves per SIMD) can issue between its own MFMAs before the matrix
// cores wait, for v_mfma_f32_16x16x32_f16 and v_mfma_f32_32x32x16_f16.  Each
// wave runs `iters` iterations of MFMAs on independent accumulators (kept in
// AGPRs and updated in place, inline asm) with V register-independent v_add_u32
// after each MFMA; the time per 16x16x32-equivalent MFMA per SIMD is reported
// (wall time; cycles at a nominal 2.1 GHz).  One block of 4 or 8 waves per CU
// (100 KB of LDS per block keeps a second block off the CU).
//
// Build and run (the GPU box): hipcc --offload-arch=gfx950 -O3 -Xclang
//   -target-feature -Xclang -packed-fp32-ops mfma_issue.hip -o mfma_issue && ./mfma_issue
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

#define VADD(r) asm volatile("v_add_u32 %0, %0, %1" : "+v"(r) : "v"(k))

template <int BIG, int V, int WAVES>
__global__ __launch_bounds__(WAVES * 64, 1) void probe(float* out, int iters) {
  __shared__ char pad[100 * 1024];  // one block per CU
  const int lane = threadIdx.x;
  u32x4_t a = u32x4_t{0x3c003c00u, 0x3c003c00u, 0x3c003c00u, (uint32_t)lane}, b = a;
  f32x4_t acc[8];
  f32x16_t acc2[4];
  for (int i = 0; i < 8; ++i) acc[i] = f32x4_t{0.f, 0.f, 0.f, 0.f};
  for (int i = 0; i < 4; ++i) acc2[i] = (f32x16_t)0.f;
  uint32_t r0 = lane, r1 = lane + 1, r2 = lane + 2, r3 = lane + 3, r4 = lane + 4, r5 = lane + 5;
  const uint32_t k = (uint32_t)iters | 1u;
  for (int it = 0; it < iters; ++it) {
    if (BIG) {
#pragma unroll
      for (int m = 0; m < 4; ++m) {
        asm volatile("v_mfma_f32_32x32x16_f16 %0, %1, %2, %0" : "+a"(acc2[m]) : "v"(a), "v"(b));
        if (V > 0) VADD(r0); if (V > 1) VADD(r1); if (V > 2) VADD(r2);
        if (V > 3) VADD(r3); if (V > 4) VADD(r4); if (V > 5) VADD(r5);
        if (V > 6) VADD(r0); if (V > 7) VADD(r1); if (V > 8) VADD(r2); if (V > 9) VADD(r3);
      }
    } else {
#pragma unroll
      for (int m = 0; m < 8; ++m) {
        asm volatile("v_mfma_f32_16x16x32_f16 %0, %1, %2, %0" : "+a"(acc[m]) : "v"(a), "v"(b));
        if (V > 0) VADD(r0); if (V > 1) VADD(r1); if (V > 2) VADD(r2);
        if (V > 3) VADD(r3); if (V > 4) VADD(r4); if (V > 5) VADD(r5);
      }
    }
  }
  // the MFMA results land before the reads below (the asm hides the MFMAs from
  // the compiler's hazard recognizer)
  asm volatile("s_nop 15\n\ts_nop 15" ::: "memory");
  float s = 0.f;
  for (int i = 0; i < 8; ++i) s += acc[i][0] + acc[i][3];
  for (int i = 0; i < 4; ++i) s += acc2[i][0] + acc2[i][15];
  s += (float)(r0 ^ r1 ^ r2 ^ r3 ^ r4 ^ r5);
  pad[lane] = (char)s;
  __syncthreads();
  out[blockIdx.x * blockDim.x + lane] = s + pad[(lane + 1) % 64];
}

template <int BIG, int V, int WAVES>
void run(float* out) {
  const int iters = 4000, blocks = 256;
  hipLaunchKernelGGL((probe<BIG, V, WAVES>), dim3(blocks), dim3(WAVES * 64), 0, 0, out, iters);
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
  (void)hipEventRecord(e0);
  hipLaunchKernelGGL((probe<BIG, V, WAVES>), dim3(blocks), dim3(WAVES * 64), 0, 0, out, iters);
  (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
  float ms; (void)hipEventElapsedTime(&ms, e0, e1);
  const double per_simd_units = (double)iters * (WAVES / 4) * 8;  // 16x16x32-equivalents per SIMD
  printf("%s waves/SIMD %d VALU per MFMA %2d: %.2f ns per 16x16x32-equivalent (%.1f cycles at 2.1 GHz)\n",
         BIG ? "32x32x16" : "16x16x32", WAVES / 4, V, ms * 1e6 / per_simd_units, ms * 1e6 / per_simd_units * 2.1);
  fflush(stdout);
}

int main() {
  float* out;
  (void)hipMalloc(&out, 256 * 512 * sizeof(float));
  run<0, 0, 4>(out); run<0, 1, 4>(out); run<0, 2, 4>(out); run<0, 3, 4>(out); run<0, 4, 4>(out);
  run<0, 0, 8>(out); run<0, 1, 8>(out); run<0, 2, 8>(out); run<0, 3, 8>(out);
  run<1, 0, 4>(out); run<1, 2, 4>(out); run<1, 4, 4>(out); run<1, 6, 4>(out); run<1, 8, 4>(out); run<1, 10, 4>(out);
  run<1, 0, 8>(out); run<1, 4, 8>(out); run<1, 6, 8>(out);
  return 0;
}
