// LDS read microbenchmark: ds_read_b128 bytes per CU per ns with 4, 8 and 16
// waves per block (one block per CU), in the access pattern of the wide-tile
// prefill kernel's fragment reads (rows of 64 halves, 16-byte chunk ch of row r
// at position ch ^ (r & 7): conflict free).
//
// Build and run (the GPU box): hipcc --offload-arch=gfx950 -O3 -Xclang
//   -target-feature -Xclang -packed-fp32-ops lds_read.hip -o lds_read && ./lds_read
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int WAVES>
__global__ __launch_bounds__(WAVES * 64, 1) void probe(uint32_t* out, int iters) {
  __shared__ __align__(16) uint16_t s[2][256 * 64];  // 64 KB: two 256 x 64-half tiles
  __shared__ char pad[40 * 1024];                       // one block per CU
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  for (int i = tid; i < 2 * 256 * 64; i += WAVES * 64) (&s[0][0])[i] = (uint16_t)i;
  pad[tid] = 1;
  __syncthreads();
  const int r = lane & 31, kh = lane >> 5;
  u32x4_t acc = u32x4_t{0u, 0u, 0u, (uint32_t)pad[(tid + 1) % 64]};
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      const int row = (wave * 32 + 8 * j + r + 8 * it) & 255, chunk = (2 * (j & 3) + kh) ^ (row & 7);
      acc ^= *reinterpret_cast<const u32x4_t*>(&s[j & 1][row * 64 + chunk * 8]);
    }
  }
  out[blockIdx.x * blockDim.x + tid] = acc[0] ^ acc[1] ^ acc[2] ^ acc[3];
}

template <int WAVES>
void run(uint32_t* out) {
  const int iters = 4000, blocks = 256;
  hipLaunchKernelGGL(probe<WAVES>, dim3(blocks), dim3(WAVES * 64), 0, 0, out, iters);
  hipEvent_t e0, e1;
  (void)hipEventCreate(&e0); (void)hipEventCreate(&e1);
  (void)hipEventRecord(e0);
  hipLaunchKernelGGL(probe<WAVES>, dim3(blocks), dim3(WAVES * 64), 0, 0, out, iters);
  (void)hipEventRecord(e1); (void)hipEventSynchronize(e1);
  float ms; (void)hipEventElapsedTime(&ms, e0, e1);
  const double bytes_per_cu = (double)iters * 16 * 1024 * WAVES;
  printf("waves %d: %.1f bytes per ns per CU (%.1f bytes per cycle at 2.1 GHz)\n", WAVES, bytes_per_cu / (ms * 1e6),
         bytes_per_cu / (ms * 1e6) / 2.1);
  fflush(stdout);
}

int main() {
  uint32_t* out;
  (void)hipMalloc(&out, 256 * 512 * sizeof(uint32_t));
  run<4>(out); run<8>(out); run<16>(out);
  return 0;
}
