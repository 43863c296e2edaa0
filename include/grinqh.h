/*
 * grinqh.h -- C ABI of libgrinqh_hip.so, the MI355X (gfx950) implementation of
 * the GRINQH quantized-linear hot path.
 *
 * Plain C: device pointers, sizes, an int status and a HIP stream passed as
 * `void*` (a hipStream_t; NULL = the default stream).  No torch or HIP types
 * appear in the signatures.  Every call only enqueues work on `stream`; none
 * synchronises the host, so all of them may be captured in a HIP graph.
 *
 * Reference paths below are relative to the otcathatsya/vllm-grinqh-plugin
 * checkout.
 *
 * Packed weight layout ("planes"): uint32 [K][Z][N/16], Z = max_bits/2, the
 * same bytes the reference's process_weights_after_loading produces
 * (grinqh/grinqh.py:200-210 -> grinqh/utils.py:17-22 and 100-146).  Word
 * (k, z, c) holds, in byte beta / slot j (bits 8*beta+7-2j .. 8*beta+6-2j), the
 * 2-bit digit z (most significant first) of W[k][(4j+beta)*(N/16) + c].
 */
#ifndef GRINQH_H_
#define GRINQH_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* status codes (0 = success) */
#define GRINQH_OK 0
#define GRINQH_ERR_INVALID 1     /* bad shape / dtype / bit width / alignment: ValueError in Python */
#define GRINQH_ERR_HIP 2         /* HIP launch error: RuntimeError in Python */
#define GRINQH_ERR_WORKSPACE 3   /* workspace missing or smaller than grinqh_workspace_bytes() */
#define GRINQH_ERR_SCRATCH 4     /* grinqh_gemm_or_gemv_noalloc: the product needs more scratch than it holds */

/* Device scratch held by the allocation-free entry point on every GPU it runs on. */
#define GRINQH_NOALLOC_SCRATCH_BYTES ((size_t)64 << 20)

/* activation / scale / output dtype */
#define GRINQH_DTYPE_F16 0
#define GRINQH_DTYPE_BF16 1

/* batch grading mode for grinqh_gemm_or_gemv */
#define GRINQH_MODE_REFERENCE 0  /* rows == 1: graded GEMV, rows > 1: dense (grinqh/kernel.py:663-680) */
#define GRINQH_MODE_UNION 1      /* every batch graded on sigma_k = max_m |x[m][k]| (grinqh/kernel.py:170-360) */
#define GRINQH_MODE_DENSE 2      /* never graded: all planes, no midpoint bias */

/* Version of this ABI (bumped on any signature or semantic change). */
int grinqh_abi_version(void);

/* Static description of a status code. */
const char* grinqh_status_string(int status);

/* Plane pack of already preshuffled + shifted codes.
 * Replaces pack_triton / _pack_kernel_uint32 (grinqh/utils.py:100-146).
 * codes_u8: uint8 [K][N] (16-byte aligned rows), planes_u32: uint32 [K][max_bits/2 * N/16].
 * N % 16 == 0, max_bits in {2,4,6,8}. */
int grinqh_pack_planes(const void* codes_u8, void* planes_u32, int64_t K, int64_t N, int max_bits,
                       void* stream);

/* Load-time preparation of a logical int8 weight W[K][N] (input-major, as the
 * weight loader leaves it): preshuffle, shift by 8-max_bits, plane pack.
 * Replaces the data path of GRINQHLinearMethod.process_weights_after_loading
 * (grinqh/grinqh.py:200-210: grinqh_input_preshuffle, <<, pack_triton). */
int grinqh_prepare_weight(const void* w_int8, void* planes_u32, int64_t K, int64_t N, int max_bits,
                          void* stream);

/* Unpack the unsigned b-bit codes of selected rows, in preshuffled column order:
 * codes_u32 is uint32 [n_rows][N/4] whose bytes are U >> (8-b).
 * Replaces unpack_pyt / unpack_triton (grinqh/utils.py:149-177, 180-223).
 * rows: int64 device array of n_rows row indices, each in [0, K) (not checked on the device).
 * bit_level = Z in 1..4. */
int grinqh_unpack_planes(const void* planes_u32, const int64_t* rows, int64_t n_rows, void* codes_u32,
                         int64_t K, int64_t N, int bit_level, void* stream);

/* Dense dequantisation in logical column order: out[k][n] = RNE(W[k][n] * scale[k/gs][n])
 * in `dtype`, or the int8 W itself when scale == NULL (out is then int8 [K][N]).
 * Replaces the unpack / sign-extend / postshuffle / scale steps of
 * grinqh_prefill_gemm_compiled (grinqh/kernel.py:568-586). */
int grinqh_dequantize(const void* planes_u32, const void* scale, void* out, int64_t K, int64_t N,
                      int max_bits, int group_size, int dtype, void* stream);

/* Grading export: zone bits (bit z = zone z active) and midpoint bias of every
 * weight row k for sigma_k = max_{m<M} |x[m][k]| (M == 1: |x[k]|), compared as
 * fp32(sigma) > thresholds[z] (strict; thresholds already rounded to fp32).
 * Replaces the inline grading of grinqh/kernel.py:98-114 (one row) and
 * :249-289 (batch union).  beta may be NULL. */
int grinqh_grade(const void* x, int64_t M, int64_t K, int64_t ldx, int dtype, int max_bits,
                 const float thresholds[4], uint8_t* zone_bits, int32_t* beta, void* stream);

/* Workspace needed by grinqh_gemm_or_gemv for this problem (0 if none): split-K
 * completion counters, fp32 split-K partial sums and, for union batches of
 * more than 16 rows, the per-row grading statistic.  From 512 rows (N a
 * multiple of 64; from 224 rows, as bf16 batches take the library GEMM from
 * there; from 257 rows when K <= 8192 or N is large enough that the fused
 * kernel would need two rounds of blocks) it also holds the dequantized
 * weight (2*N*K bytes) that the library GEMM multiplies, after the fused
 * kernel's regions (a shape the library has no algorithm for runs the
 * hand-written prefill kernels from the same workspace).  It must be zero-filled once before its
 * first use (every call leaves its counters zero again; the rest needs no
 * initial contents), 256-byte aligned, and calls that share it must be
 * ordered (same stream). */
size_t grinqh_workspace_bytes(int64_t M, int64_t K, int64_t N, int max_bits, int mode);

/* The quantized linear y[M][N] = x[M][K] * W_eff (+ bias), x/scale/bias/y in `dtype`.
 * Replaces torch.ops.grinqh.gemm_or_gemv (grinqh/kernel.py:646-710); N here is
 * 4 * original_n.  thresholds: 4 fp32 values (zero padded like
 * grinqh/grinqh.py:111).  x rows are ldx elements apart (ldx % 8 == 0, x
 * 16-byte aligned), y is dense [M][N] (8-byte aligned).  K % 32 == 0,
 * N % 16 == 0, group_size % 32 == 0. */
int grinqh_gemm_or_gemv(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                        const void* planes_u32, const void* scale, const void* bias, void* y,
                        int max_bits, int group_size, const float thresholds[4], int mode,
                        void* workspace, size_t workspace_bytes, void* stream);

/* Batch-union GEMV: grinqh_gemm_or_gemv with GRINQH_MODE_UNION.
 * Replaces grinqh_gemv_batch_union (grinqh/kernel.py:607-643). */
int grinqh_gemv_batch_union(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                            const void* planes_u32, const void* scale, const void* bias, void* y,
                            int max_bits, int group_size, const float thresholds[4],
                            void* workspace, size_t workspace_bytes, void* stream);

/* Dense dequantize-then-matmul for any M: grinqh_gemm_or_gemv with GRINQH_MODE_DENSE.
 * Replaces grinqh_prefill_gemm_compiled (grinqh/kernel.py:561-587) and, for
 * max_bits == 4, the Marlin path (grinqh/kernel.py:528-558). */
int grinqh_prefill_dense(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                         const void* planes_u32, const void* scale, const void* bias, void* y,
                         int max_bits, int group_size, void* workspace, size_t workspace_bytes,
                         void* stream);

/* ---- Producer fusion: the operations that feed a GRINQH linear also emit
 * the union statistic sigma_k = max_m |y[m][k]| its grading needs
 * (grinqh/kernel.py:249), as column maxima of row chunks: sigma_chunks is
 * float [ceil(M / GRINQH_SIGMA_CHUNK_ROWS)][K], the maximum over its chunks is
 * sigma_k (NaN ignored unless every value is NaN).  No counterpart in the
 * reference, whose grading reads x again inside the GEMV. */
#define GRINQH_SIGMA_CHUNK_ROWS 16

/* y = RNE(h * rsqrt(mean_k(h^2) + eps)) * weight with h = x, or, when residual
 * is given, h = RNE(x + residual) written to residual_out (vLLM's
 * fused_add_rms_norm arithmetic).  x [M][ldx], residual / residual_out / y
 * [M][K] dense, weight [K]; all 16-byte aligned, K % 8 == 0.  y must not
 * overlap x or residual, nor residual_out residual. */
int grinqh_rmsnorm_sigma(const void* x, int64_t M, int64_t K, int64_t ldx, const void* residual, void* residual_out,
                         const void* weight, float eps, void* y, float* sigma_chunks, int dtype, void* stream);

/* y[m][f] = RNE(silu(g)) * u with gate_up rows [g (F values) | u (F values)]
 * ld elements apart (vLLM's SiluAndMul arithmetic); y [M][F] dense, must not
 * overlap gate_up; F % 8 == 0, 16-byte aligned. */
int grinqh_silu_mul_sigma(const void* gate_up, int64_t M, int64_t F, int64_t ld, void* y, float* sigma_chunks,
                          int dtype, void* stream);

/* grinqh_gemv_batch_union grading from the sigma_chunks a producer wrote for
 * this x (ceil(M / GRINQH_SIGMA_CHUNK_ROWS) arrays of K floats) instead of
 * reading x for it: batches of 17-64 rows skip the statistic pass.  Larger
 * batches (prefill) compute their own statistic and ignore sigma_chunks.
 * Same workspace as grinqh_gemm_or_gemv in GRINQH_MODE_UNION. */
int grinqh_gemv_batch_union_sigma(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                                  const void* planes_u32, const void* scale, const void* bias, void* y,
                                  int max_bits, int group_size, const float thresholds[4],
                                  const float* sigma_chunks, void* workspace, size_t workspace_bytes,
                                  void* stream);

/* Allocation-free quantized linear.  No counterpart in the reference: it is
 * for callers that cannot allocate device memory (code under HIP graph
 * capture, tight serving loops, harnesses that forbid hipMalloc).  Same
 * arguments, semantics and results as grinqh_gemm_or_gemv, without the
 * workspace: its split-K counters, partial sums and grading statistic live in
 * a fixed device array of GRINQH_NOALLOC_SCRATCH_BYTES (64 MiB) that each GPU
 * holds from the first call until the process ends.  It calls no allocator
 * of its own (no hipMalloc, hipFree or allocating library routine).  A few
 * kernel instantiations spill registers to the private-segment (scratch)
 * memory that the HIP runtime sets up for a device's queues (the large-batch
 * kernel's 512-row blocks: tests check the build's resource report); a
 * caller that must see no runtime allocation at
 * all runs one call of each shape class first.  The library-GEMM prefill path
 * (a 2*N*K dense weight buffer) is not taken: from 256 rows the hand-written
 * large-batch kernel runs where its repacked activations fit the array, else
 * the fused kernels; a decode batch whose split-K partial sums would outgrow
 * the array runs in row chunks graded on the whole batch's statistic.  A
 * product that still does not fit (a fused prefill with many K ranges)
 * returns GRINQH_ERR_SCRATCH.  All calls on one
 * GPU share the array, so calls that overlap in time on one GPU (different
 * streams, or several threads) race; calls ordered on one stream do not.
 * The device current in the calling thread must be the one that holds the
 * pointers and the stream. */
int grinqh_gemm_or_gemv_noalloc(const void* x, int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype,
                                const void* planes_u32, const void* scale, const void* bias, void* y,
                                int max_bits, int group_size, const float thresholds[4], int mode,
                                void* stream);

/* Benchmark instrumentation; no counterpart in the reference.  Arms a one-shot
 * timer: in the next grinqh_gemm_or_gemv / grinqh_gemv_batch_union /
 * grinqh_prefill_dense call (from any thread), the dispatch of its first main
 * kernel records `event_before` as the kernel starts and `event_after` as it
 * ends (hipExtLaunchKernelGGL), so the events time that kernel's execution
 * alone: no split-K reduction, no event or dispatch overhead.  Both are
 * hipEvent_t handles created by the caller with timing enabled; passing two
 * NULLs disarms.  Not for use under graph capture. */
int grinqh_time_next_product(void* event_before, void* event_after);

/* Kernel selection query; no counterpart in the reference (for tests and
 * benchmarks).  Names the kernel that serves an M-row product of this shape
 * through grinqh_gemm_or_gemv (noalloc = 0) or grinqh_gemm_or_gemv_noalloc
 * (noalloc = 1), nothing launched: GRINQH_KERNEL_GEMV (1-4 rows per launch),
 * GRINQH_KERNEL_DECODE (5-64), GRINQH_KERNEL_TALL (the large-batch prefill;
 * *rows_per_block and *splits receive its plan), GRINQH_KERNEL_LIBRARY (the
 * dense weight and the library GEMM, where the dispatch prefers it; the
 * library's algorithm query at run time can still send the call to the fused
 * prefill) or GRINQH_KERNEL_FUSED (the fused prefill).  GRINQH_PREFILL=tall or
 * =library in the environment forces the large-batch kernel or the library
 * path where they apply, as for the products.  Returns the kernel id, or a
 * negative status for bad arguments. */
#define GRINQH_KERNEL_GEMV 1
#define GRINQH_KERNEL_DECODE 2
#define GRINQH_KERNEL_TALL 3
#define GRINQH_KERNEL_LIBRARY 4
#define GRINQH_KERNEL_FUSED 5
int grinqh_product_kernel(int64_t M, int64_t K, int64_t ldx, int64_t N, int dtype, int max_bits, int group_size,
                          int mode, int noalloc, int* rows_per_block, int* splits);

#ifdef __cplusplus
}
#endif

#endif /* GRINQH_H_ */
