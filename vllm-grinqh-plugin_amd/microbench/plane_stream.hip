// Plane-streaming microbenchmark: how fast can gfx950 read a GRINQH plane
// array [K][Z][N/16] (uint32 words, the reference layout) in the access
// patterns the product kernels use, with no arithmetic besides an XOR of the
// words?  It answers whether the reference layout itself limits the decode
// kernels, or whether a repacked layout would read faster.
//
// Shape: Llama-3-8B gate_up (K = 4096, N = 28672, max_bits 8: Z = 4 planes,
// NW = 1792 words per plane row), 117 MB per copy.  Four copies are rotated
// (470 MB, more than the 256 MB MALL), so every launch reads from HBM.
// "graded": rows use 1/2/3/4 planes with probability 0.5/0.3/0.15/0.05 (the
// threshold mix of the benchmark), and a plane a row does not use is not read
// (its load offset is out of range: the buffer load returns 0 without a memory
// access).  GB/s counts the bytes of the planes used.
//
// Patterns (each lane XORs the words it loads; one dword load per plane word):
//   blk16    the decode kernel's mapping: a block = 16 word columns, lane
//            (c, q) = word column c, rows 8q..8q+7 of a 32-row tile; the 4
//            waves take consecutive K sub-ranges.  Two neighbouring blocks
//            share every 128-byte line.
//   col64    4 waves on 4 adjacent 16-word column groups (64 word columns per
//            block, whole 256-byte runs per block), same lane roles.
//   row64    the GEMV kernel's mapping: lane = word column (64 per wave), one
//            (row, plane) run of 256 bytes per load; 4 waves = K sub-ranges.
//   tiled    a repacked layout [N/256][K/32][Z][32][16] (each block's tile is
//            contiguous), lane roles of blk16.
// Each at one and two blocks of 4 waves per CU.
//
// Build and run (the GPU box): hipcc --offload-arch=gfx950 -O3 -std=c++17
//   -Xclang -target-feature -Xclang -packed-fp32-ops plane_stream.hip -o plane_stream && ./plane_stream
#include <hip/hip_runtime.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>

namespace {

constexpr int Z = 4;
constexpr int K = 4096;
constexpr int NW = 1792;  // N / 16
constexpr int T = K / 32;
constexpr size_t kWords = (size_t)K * Z * NW;
constexpr uint32_t kNone = 0x80000000u;  // out-of-range offset: the load returns 0, no memory access

enum Pattern { BLK16, COL64, ROW64, TILED };

// Byte offset of plane word (row, z, word column w) in the pattern's layout.
template <int PAT>
__device__ __forceinline__ uint32_t word_offset(int row, int z, int w) {
  if constexpr (PAT == TILED) {
    const int cb = w >> 4, c = w & 15, t = row >> 5, r = row & 31;
    return (uint32_t)((((((size_t)cb * T + t) * Z + z) * 32 + r) * 16 + c) * 4);
  } else {
    return (uint32_t)((((size_t)row * Z + z) * NW + w) * 4);
  }
}

// One block: 4 waves.  BLK16/TILED: 16 word columns, waves = K sub-ranges of
// the block's rows.  COL64: 64 word columns, wave = 16-column group, all rows
// of the block's range.  ROW64: 64 word columns, lane = column, waves = K
// sub-ranges.  Three tiles of loads per wave in flight (two ahead).
template <int PAT, int OCC>
__global__ __launch_bounds__(256, OCC) void stream(const uint32_t* __restrict__ P, const uint8_t* __restrict__ zones,
                                                   int tiles_per_block, uint32_t* __restrict__ out) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int c = lane & 15, q = lane >> 4;
  const int t0 = blockIdx.y * tiles_per_block, t1 = min(t0 + tiles_per_block, T);
  const int nt = t1 - t0;
  int tb, te, wcol;
  if constexpr (PAT == COL64) {
    tb = t0, te = t1, wcol = blockIdx.x * 64 + wave * 16 + c;
  } else {
    tb = t0 + nt * wave / 4, te = t0 + nt * (wave + 1) / 4;
    wcol = PAT == ROW64 ? blockIdx.x * 64 + lane : blockIdx.x * 16 + c;
  }
  const __amdgpu_buffer_rsrc_t rs =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<uint32_t*>(P), (short)0, (int)(kWords * 4), 0x00020000);
  uint32_t acc = 0;
  // per tile and lane: 8 rows x Z planes (ROW64: 8 rows of the wave's 32-row tile quarter... all 32 rows in 4 steps)
  uint32_t DA[8][Z], DB[8][Z], DC[8][Z];
  auto issue = [&](int t, int part, uint32_t (&D)[8][Z]) {
    const bool live = t < te;
    const int tt = live ? t : tb;
    for (int e = 0; e < 8; ++e) {
      // ROW64: one tile is 4 parts of 8 rows, every lane on the same row; others: rows 8q + e
      const int row = PAT == ROW64 ? tt * 32 + 8 * part + e : tt * 32 + 8 * q + e;
      const uint32_t bits = zones[row];
      for (int z = 0; z < Z; ++z) {
        const bool on = live && ((bits >> z) & 1u);
        D[e][z] = __builtin_amdgcn_raw_buffer_load_b32(rs, (int)(on ? word_offset<PAT>(row, z, wcol) : kNone), 0, 0);
      }
    }
  };
  auto use = [&](uint32_t (&D)[8][Z]) {
    for (int e = 0; e < 8; ++e)
      for (int z = 0; z < Z; ++z) acc ^= D[e][z] + (uint32_t)e;
  };
  // steps: (tile, part) pairs; ROW64 has 4 parts per tile, the others 1
  constexpr int PARTS = PAT == ROW64 ? 4 : 1;
  const int steps = (te - tb) * PARTS;
  auto at = [&](int s, uint32_t (&D)[8][Z]) { issue(tb + s / PARTS, s % PARTS, D); };
  at(0, DA);
  at(1, DB);
  int s = 0;
  for (; s + 3 <= steps; s += 3) {
    at(s + 2, DC); __builtin_amdgcn_sched_barrier(0); use(DA);
    at(s + 3, DA); __builtin_amdgcn_sched_barrier(0); use(DB);
    at(s + 4, DB); __builtin_amdgcn_sched_barrier(0); use(DC);
  }
  if (s < steps) use(DA);
  if (s + 1 < steps) use(DB);
  out[((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 256 + threadIdx.x] = acc;
}

#define CK(x)                                                                          \
  do {                                                                                 \
    hipError_t e_ = (x);                                                               \
    if (e_ != hipSuccess) {                                                            \
      printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);            \
      exit(1);                                                                         \
    }                                                                                  \
  } while (0)

}  // namespace

int main() {
  const int copies = 4;
  uint32_t* P;
  uint32_t* out;
  uint8_t *z_full, *z_graded;
  CK(hipMalloc(&P, kWords * 4 * copies));
  CK(hipMemset(P, 0x5A, kWords * 4 * copies));
  CK(hipMalloc(&out, (size_t)NW / 16 * T * 256 * 4));
  CK(hipMalloc(&z_full, K));
  CK(hipMalloc(&z_graded, K));
  static uint8_t h_full[K], h_gr[K];
  srand(1);
  double planes = 0;
  for (int k = 0; k < K; ++k) {
    h_full[k] = 15;
    const double u = rand() / (double)RAND_MAX;
    h_gr[k] = u < 0.5 ? 1 : (u < 0.8 ? 3 : (u < 0.95 ? 7 : 15));
    planes += __builtin_popcount(h_gr[k]);
  }
  const double frac = planes / (4.0 * K);
  CK(hipMemcpy(z_full, h_full, K, hipMemcpyHostToDevice));
  CK(hipMemcpy(z_graded, h_gr, K, hipMemcpyHostToDevice));
  hipEvent_t e0, e1;
  CK(hipEventCreate(&e0));
  CK(hipEventCreate(&e1));
  printf("gate_up planes: K=%d NW=%d Z=%d, %.1f MB per copy, %d copies rotated; graded plane fraction %.3f\n", K, NW,
         Z, kWords * 4 / 1e6, copies, frac);
  printf("%-8s %-4s %-6s %6s %9s %9s\n", "pattern", "occ", "planes", "blocks", "us", "GB/s");
  auto run = [&](const char* name, auto kern, int occ, int cols_per_block, int splits, bool graded) {
    const int tpb = (T + splits - 1) / splits;
    const dim3 grid(NW / cols_per_block, (T + tpb - 1) / tpb);
    // every offset is below kWords * 4: rows < K, word columns < NW (NW % 64 == 0)
    auto launch = [&](int r) {
      hipLaunchKernelGGL(kern, grid, dim3(256), 0, 0, P + (size_t)r * kWords, graded ? z_graded : z_full, tpb, out);
    };
    for (int w = 0; w < 2; ++w) launch(w % copies);
    CK(hipDeviceSynchronize());
    const int reps = 40;
    CK(hipEventRecord(e0));
    for (int r = 0; r < reps; ++r) launch(r % copies);
    CK(hipEventRecord(e1));
    CK(hipEventSynchronize(e1));
    float ms;
    CK(hipEventElapsedTime(&ms, e0, e1));
    const double us = ms * 1e3 / reps;
    const double bytes = kWords * 4.0 * (graded ? frac : 1.0);
    printf("%-8s %-4d %-6s %6u %9.2f %9.0f\n", name, occ, graded ? "graded" : "all", grid.x * grid.y, us,
           bytes / (us * 1e-6) / 1e9);
    fflush(stdout);
  };
  for (bool g : {false, true}) {
    run("blk16", stream<BLK16, 1>, 1, 16, 2, g);
    run("blk16", stream<BLK16, 2>, 2, 16, 4, g);
    run("tiled", stream<TILED, 1>, 1, 16, 2, g);
    run("tiled", stream<TILED, 2>, 2, 16, 4, g);
    run("col64", stream<COL64, 1>, 1, 64, 9, g);
    run("col64", stream<COL64, 2>, 2, 64, 16, g);
    run("row64", stream<ROW64, 1>, 1, 64, 9, g);
    run("row64", stream<ROW64, 2>, 2, 64, 16, g);
  }
  return 0;
}
