// Shared device helpers for the GRINQH gfx950 kernels.
//
// Weight layout (identical bytes to the reference's packed parameter, produced
// by process_weights_after_loading in grinqh/grinqh.py:200-210 of the
// reference): uint32 planes[K][Z][NW] with NW = N/16.  Word (k, z, c) holds,
// in byte beta / slot j (bits 8*beta+7-2j .. 8*beta+6-2j), the 2-bit digit z
// (most significant first) of logical column n = (4j+beta)*NW + c of row k.
//
// A lane that owns word column c therefore sees 16 logical columns at once,
// one per "column tile" r = 4j+beta; tile r of a 16-word block w0..w0+15 is the
// 16 contiguous columns r*NW + w0 .. r*NW + w0 + 15.  This is what maps the
// plane words straight onto the B operand of v_mfma_f32_16x16x32_{f16,bf16}
// (lane = column-in-tile + 16*k_octet, 8 consecutive k per lane).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace grinqh {

typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));

struct F16 { static constexpr int id = 0; };
struct BF16 { static constexpr int id = 1; };

// ---------------------------------------------------------------- scalars

__device__ __forceinline__ float f16_bits_to_f32(uint16_t h) {
  _Float16 v;
  __builtin_memcpy(&v, &h, 2);
  return (float)v;
}
__device__ __forceinline__ float bf16_bits_to_f32(uint16_t h) {
  return __uint_as_float(((uint32_t)h) << 16);
}
__device__ __forceinline__ uint16_t f32_to_f16_bits(float f) {
  _Float16 v = (_Float16)f;  // v_cvt_f16_f32, round to nearest even
  uint16_t h;
  __builtin_memcpy(&h, &v, 2);
  return h;
}
__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
  uint32_t u = __float_as_uint(f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((u >> 16) | 0x40u);  // quiet NaN
  u += 0x7fffu + ((u >> 16) & 1u);  // round to nearest even
  return (uint16_t)(u >> 16);
}

template <typename DT> __device__ __forceinline__ float to_f32(uint16_t h);
template <> __device__ __forceinline__ float to_f32<F16>(uint16_t h) { return f16_bits_to_f32(h); }
template <> __device__ __forceinline__ float to_f32<BF16>(uint16_t h) { return bf16_bits_to_f32(h); }
template <typename DT> __device__ __forceinline__ uint16_t from_f32(float f);
template <> __device__ __forceinline__ uint16_t from_f32<F16>(float f) { return f32_to_f16_bits(f); }
template <> __device__ __forceinline__ uint16_t from_f32<BF16>(float f) { return f32_to_bf16_bits(f); }

// Output epilogue shared by every product kernel: the reference casts the fp32
// result to the activation dtype and then adds the bias in that dtype
// (grinqh/kernel.py:706-708), i.e. two roundings.
template <typename DT>
__device__ __forceinline__ uint16_t finish_output(float acc, const uint16_t* bias, int n) {
  uint16_t y = from_f32<DT>(acc);
  if (bias != nullptr) y = from_f32<DT>(to_f32<DT>(y) + to_f32<DT>(bias[n]));
  return y;
}

// Graded (union) products that multiply the scaled weight w_eff * s directly:
// a sum that is not finite can only come from a non-finite activation in its
// row (fp16/bf16 products cannot overflow fp32), and every output of such a
// row is then non-finite.  The reference keeps the midpoint-bias term apart,
// sum_k beta_k * x_k * s (grinqh/kernel.py:113-114, 148-158), whose 0 * inf or
// 0 * NaN makes the whole row NaN; mapping each non-finite sum to NaN gives
// that row.
__device__ __forceinline__ float graded_nonfinite_to_nan(float v) {
  return __builtin_isfinite(v) ? v : __builtin_nanf("");
}

// ---------------------------------------------------------------- bytes

// v_perm_b32: byte selector 0..3 picks from `lo`, 4..7 from `hi`, 0x0c gives 0.
__device__ __forceinline__ uint32_t perm(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
__device__ __forceinline__ uint32_t rotr(uint32_t v, uint32_t r) {
  return __builtin_amdgcn_alignbit(v, v, r);
}

// ---------------------------------------------------------------- MFMA

template <typename DT>
__device__ __forceinline__ f32x4_t mfma16x16x32(const u32x4_t& a, const u32x4_t& b, f32x4_t c);
template <>
__device__ __forceinline__ f32x4_t mfma16x16x32<F16>(const u32x4_t& a, const u32x4_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(half8_t, a),
                                                __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mfma16x16x32<BF16>(const u32x4_t& a, const u32x4_t& b, f32x4_t c) {
  return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                 __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
}

// v_mfma_f32_16x16x16_{f16,bf16}: lane (c, q) holds A[c][4q..4q+3] and
// B[4q..4q+3][c]; D as for 16x16x32.
template <typename DT>
__device__ __forceinline__ f32x4_t mfma16x16x16(const u32x2_t& a, const u32x2_t& b, f32x4_t c);
template <>
__device__ __forceinline__ f32x4_t mfma16x16x16<F16>(const u32x2_t& a, const u32x2_t& b, f32x4_t c) {
  typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(half4_t, a), __builtin_bit_cast(half4_t, b), c,
                                               0, 0, 0);
}
template <>
__device__ __forceinline__ f32x4_t mfma16x16x16<BF16>(const u32x2_t& a, const u32x2_t& b, f32x4_t c) {
  typedef short short4_t __attribute__((ext_vector_type(4)));
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(short4_t, a), __builtin_bit_cast(short4_t, b),
                                                   c, 0, 0, 0);
}

// ---------------------------------------------------------------- block order

// The workgroups of a launch are dealt to the 8 XCDs round robin (linear id
// mod 8), and each XCD has its own L2.  xcd_chunked renumbers linear id L of
// `total` workgroups so that every XCD runs one contiguous range of logical
// blocks: logical neighbours (column blocks that share 128-byte lines) meet in
// one L2 instead of each XCD fetching the whole line.  A bijection on
// [0, total) for any total.
__device__ __forceinline__ int xcd_chunked(int L, int total) {
  constexpr int kXcds = 8;
  const int per = total / kXcds, rem = total % kXcds;
  const int xcd = L % kXcds, slot = L / kXcds;
  return xcd < rem ? xcd * (per + 1) + slot : rem * (per + 1) + (xcd - rem) * per + slot;
}

// ---------------------------------------------------------------- grading

// sigma_k = max_m |x[m][k]| with NaN ignored (fmaxf) unless every entry is NaN.
// Loads are issued in batches of 8 independent, clamped (in-bounds) addresses.
template <typename DT>
__device__ __forceinline__ float column_absmax(const uint16_t* __restrict__ x, int64_t ldx, int M, int k) {
  float s = fabsf(to_f32<DT>(x[k]));
  for (int m0 = 1; m0 < M; m0 += 8) {
    uint16_t v[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) v[i] = x[(int64_t)min(m0 + i, M - 1) * ldx + k];
#pragma unroll
    for (int i = 0; i < 8; ++i) s = fmaxf(s, fabsf(to_f32<DT>(v[i])));
  }
  return s;
}


// Zone bits of one row statistic: bit z set iff z < Z and fp32(|sigma|) > t_z
// (strict, NaN false), the Triton fp32 promotion of grinqh/kernel.py:100-106.
template <int Z>
__device__ __forceinline__ uint32_t zone_bits(float sigma_abs, const float* thr) {
  uint32_t b = 0;
#pragma unroll
  for (int z = 0; z < Z; ++z) b |= (sigma_abs > thr[z]) ? (1u << z) : 0u;
  return b;
}

// Midpoint bias beta of an arbitrary zone set: sum of the telescoped deltas
// Delta_0 = B>>2, Delta_z = (B>>(2z+2)) - (B>>2z), B = 1<<(b-1)
// (grinqh/kernel.py:73-82, 108-113).
template <int Z>
__device__ __forceinline__ int midpoint_bias(uint32_t bits) {
  constexpr int B = 1 << (2 * Z - 1);
  int beta = 0, prev = 0;
#pragma unroll
  for (int z = 0; z < Z; ++z) {
    const int cur = B >> (2 * z + 2);
    if ((bits >> z) & 1u) beta += cur - prev;
    prev = cur;
  }
  return beta;
}

// Grade word of one K row for kernels that dequantize whole rows of a graded
// batch (the large-batch prefill): the zone set of sigma_k in bits 16 .. 16 +
// Z - 1, and in the low half the row constant of the dequantization with
// sh = 8 - 2 Z: for fp16 activations -(1024 + (128 >> sh) - beta) as fp16
// (added to 1024 + (u >> sh)), for bf16 the integer c_row = 128 - beta * 2^sh
// (subtracted from u).  The same zone set and midpoint bias as zone_bits /
// midpoint_bias of sigma_k, computed once per row instead of once per block.
template <typename DT, int Z>
__device__ __forceinline__ uint32_t grade_word(float sigma_abs, const float* thr) {
  constexpr int SH = 8 - 2 * Z;
  const uint32_t bits = zone_bits<Z>(sigma_abs, thr);
  const int beta = midpoint_bias<Z>(bits);
  uint32_t lo;
  if constexpr (DT::id == F16::id)
    lo = f32_to_f16_bits(-(float)(1024 + (128 >> SH) - beta));
  else
    lo = (uint32_t)(uint16_t)(int16_t)(128 - beta * (1 << SH));
  return lo | (bits << 16);
}

// ---------------------------------------------------------------- unpack

// Bit-field insert: bits of `a` where `m` is set, bits of `b` elsewhere, in the
// bit-select form the backend turns into v_bfi_b32 where it can.  It must stay
// ordinary code: the compiler inserts the wait states an MFMA's result write
// needs before a later VALU write of the same register only for instructions
// it can see.  As inline asm this was not done, and a v_bfi_b32 that reused a
// register of an in-flight MFMA's unused result elements (the one-row GEMV's
// accumulators have three) was overwritten when the MFMA's write landed last.
__device__ __forceinline__ uint32_t bfi(uint32_t m, uint32_t a, uint32_t b) { return ((a ^ b) & m) ^ b; }

// Code-byte rebuild for 8 rows of plane words D[e][z] (one word per plane).
// Plane z's digit of slot j sits in field 3-j of each byte (bits 8*beta+6-2j).
// prepare_planes flips zone 0's top digit bit where zone 0 is active (offset
// binary: the byte becomes int8(U & mask) + 128) and rotates
// G_z = rot(D_z, 2z), which moves slot j's digit to field (3-z-j)&3; then
// code_dwords merges field (3-z-j)&3 of every G_z (the fields are disjoint)
// and rotates back: V_j = rot(H_j, -2j) holds the code bytes of column tiles
// 4j+beta, digit z in field 3-z.
// xm[e] is the zone-0 flip of row e: 0xAAAAAAAA when zone 0 is active (the
// byte is then int8(U & mask) + 128), 0 otherwise (the byte is U & mask, which
// has bit 7 clear).  A row with no active zone thus rebuilds to exact zeros.
template <int Z, int E = 8>
__device__ __forceinline__ void prepare_planes(uint32_t (&D)[E][Z], const uint32_t (&xm)[E]) {
#pragma unroll
  for (int e = 0; e < E; ++e) {
    D[e][0] ^= xm[e];
#pragma unroll
    for (int z = 1; z < Z; ++z) D[e][z] = rotr(D[e][z], (uint32_t)(2 * z));
  }
}
__device__ __forceinline__ uint32_t zone0_flip(uint32_t bits) { return (bits & 1u) ? 0xAAAAAAAAu : 0u; }
template <int Z, int E = 8>
__device__ __forceinline__ void code_dwords(const uint32_t (&G)[E][Z], int j, uint32_t (&V)[E]) {
#pragma unroll
  for (int e = 0; e < E; ++e) {
    // with all four planes the last one fills the remaining field, otherwise
    // the fields no plane owns are zero
    uint32_t h = (Z == 4) ? G[e][3] : (G[e][0] & (0x03030303u << (2 * ((3 - j) & 3))));
#pragma unroll
    for (int z = (Z == 4 ? 0 : 1); z < (Z == 4 ? 3 : Z); ++z)
      h = bfi(0x03030303u << (2 * ((3 - z - j) & 3)), G[e][z], h);
    V[e] = rotr(h, (uint32_t)(32 - 2 * j) & 31u);
  }
}

// ---------------------------------------------------------------- MFMA B operand

// B registers of v_mfma_f32_16x16x32_{f16,bf16} from rebuilt code bytes: V[e]
// holds the offset-binary code bytes of row e (byte beta = column tile
// 4j+beta); B[beta][p] holds rows 2p, 2p+1 of column tile beta.
template <typename DT>
struct BOperand;

// fp16: B = u as a subnormal, u * 2^-24 (exact: u < 2^10); built with one
// v_perm per register from the code bytes of two consecutive rows.
template <>
struct BOperand<F16> {
  static constexpr float kUnit = 16777216.f;  // 2^24: undoes the subnormal scaling
  __device__ __forceinline__ static void build(const uint32_t (&V)[8], u32x4_t (&B)[4]) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int beta = 0; beta < 4; ++beta) B[beta][p] = pair(V[2 * p], V[2 * p + 1], beta);
  }
  // rows e0 (low half) and e1 (high half) of column tile beta
  __device__ __forceinline__ static uint32_t pair(uint32_t v0, uint32_t v1, int beta) {
    return perm(v1, v0, 0x0C040C00u + (uint32_t)beta * 0x00010001u);
  }
  __device__ __forceinline__ static uint16_t correction(int v) {  // v * 2^-24, |v| < 1024
    return v >= 0 ? (uint16_t)v : (uint16_t)(0x8000u | (uint32_t)(-v));
  }
};

// bf16: B = u (0..255 has at most 8 significant bits, exact in bf16).
template <>
struct BOperand<BF16> {
  static constexpr float kUnit = 1.f;
  __device__ __forceinline__ static void build(const uint32_t (&V)[8], u32x4_t (&B)[4]) {
#pragma unroll
    for (int p = 0; p < 4; ++p)
#pragma unroll
      for (int beta = 0; beta < 4; ++beta) B[beta][p] = pair(V[2 * p], V[2 * p + 1], beta);
  }
  __device__ __forceinline__ static uint32_t pair(uint32_t v0, uint32_t v1, int beta) {
    const float a = (float)((v0 >> (8 * beta)) & 0xFFu);
    const float b = (float)((v1 >> (8 * beta)) & 0xFFu);
    return perm(__float_as_uint(b), __float_as_uint(a), 0x07060302u);
  }
  __device__ __forceinline__ static uint16_t correction(int v) { return from_f32<BF16>((float)v); }
};

// ---------------------------------------------------------------- dequantised operand

typedef _Float16 half2_t __attribute__((ext_vector_type(2)));

// Two rows (low half = row 0, high half = row 1) of column tile beta from the
// code dwords V0, V1 (offset-binary bytes u) as the scaled weight RNE(w * s)
// in the activation dtype, with w = (u >> sh) - c_row and the per-row constant
// c_row = 1024 + (offset 128 >> sh of an offset-binary row) - beta_row.
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
  // the same with s = half `hi` of sp (two columns' scales): the broadcast
  // folds into the packed multiply's operand select, so no register holds
  // the (s, s) pair
  __device__ __forceinline__ static uint32_t pair_half(uint32_t V0, uint32_t V1, int beta, uint32_t negc, uint32_t sp,
                                                       int hi) {
    const _Float16 s = __builtin_bit_cast(half2_t, sp)[hi];
    return pair(V0, V1, beta, negc, __builtin_bit_cast(uint32_t, half2_t{s, s}));
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

}  // namespace grinqh
