"""CPU oracle for the GRINQH quantized-linear hot path.

TEST INFRASTRUCTURE ONLY.  Only ``tests/``, ``__graft_entry__.smoke()`` and the
``cpu_baseline`` leg of ``bench.py`` may import this module, and only as the
checker.  The product (``grinqh`` package + ``libgrinqh_hip.so``) never imports,
links or falls back to it.

Every function restates one step of the reference algorithm in numpy and cites
the reference file:line it follows (paths relative to the reference checkout of
otcathatsya/vllm-grinqh-plugin).  Notation: ``K`` = in_features (rows of the
input-major weight), ``N`` = out_features, ``b`` = max_bits in {2,4,6,8},
``Z = b/2`` bit-planes ("zones"), ``sh = 8-b``.

Parity pins (each function is checked in tests/test_oracle.py against something
other than itself):

* ``preshuffle``/``postshuffle``   -- inverse pair + explicit index formula.
* ``pack_planes``                  -- storage-size identity (tests/test_grinqh_ops.py:76),
                                      round trip ``unpack(pack(A)) == A >> sh`` (:87-88),
                                      independent index derivation from the Marlin
                                      converter (grinqh/kernel.py:393-398).
* ``unpack_planes``                -- vectorised == per-row (:82-85) and the round trip.
* ``grade``                        -- Triton fp32 promotion rule (|x| and t in fp32,
                                      strict ``>``), special cases t=-1 (all zones)
                                      and quantile 1.0 (no zone), brute force over all
                                      fp16 values against a threshold pair.
* ``union_sigma``                  -- NaN rule of Triton's ``tl.max`` read from the
                                      installed Triton (3.6.0; the reference pins 3.7.1,
                                      uv.lock:5094), padding rule brute-forced on tiny batches.
* ``effective_weight``             -- closed form ``floor(c / 2^(b-2a)) * 2^(b-2a) + 2^(b-2a-1)``
                                      for prefix masks, and the reference test oracle's
                                      dense form (tests/test_grinqh_ops.py:28-55).
* ``gemv``/``gemv_union``/``dense_prefill`` -- reference test identities (all-active
                                      GEMV == dense fp32 matmul, union == looped GEMV
                                      at all-active thresholds, skip_all == 0).
"""
from __future__ import annotations

import numpy as np

__all__ = [
    "preshuffle", "postshuffle", "shift_codes", "pack_planes", "unpack_planes",
    "prepare_weight", "grade", "union_sigma", "zone_mask_byte", "midpoint_bias", "effective_weight",
    "masked_weight_ref", "gemv_f64", "gemv", "gemv_union_f64", "gemv_union",
    "dense_prefill", "dense_prefill_f64", "gemm_or_gemv", "to_f32_threshold",
    "rne_cast", "bias_add",
]


# ----------------------------------------------------------------------------
# S2 / S3 / S4 / S5 : layout
# ----------------------------------------------------------------------------

def preshuffle(w: np.ndarray) -> np.ndarray:
    """S2. ``P[k, 16c + r] = W[k, r*(N/16) + c]`` (grinqh/utils.py:17-22)."""
    K, N = w.shape
    if N % 16 != 0:
        raise AssertionError("N must be divisible by 16 for this layout.")
    return np.ascontiguousarray(w.reshape(K, 16, N // 16).transpose(0, 2, 1)).reshape(K, N)


def postshuffle(w: np.ndarray) -> np.ndarray:
    """Inverse of S2 (grinqh/utils.py:25-30)."""
    K, N = w.shape
    if N % 16 != 0:
        raise AssertionError("N must be divisible by 16 for this layout.")
    return np.ascontiguousarray(w.reshape(K, N // 16, 16).transpose(0, 2, 1)).reshape(K, N)


def shift_codes(w_int8: np.ndarray, max_bits: int) -> np.ndarray:
    """S3. ``U = uint8(W << (8-b))`` (grinqh/grinqh.py:204-205)."""
    sh = 8 - max_bits
    return ((np.asarray(w_int8, dtype=np.int8).view(np.uint8).astype(np.uint16) << sh) & 0xFF).astype(np.uint8)


def pack_planes(U: np.ndarray, max_bits: int) -> np.ndarray:
    """S4. Bit-plane pack of uint8 ``U[K, N]`` into uint32 ``[K, Z*N/16]``.

    Follows ``_pack_kernel_uint32`` / ``pack_triton`` (grinqh/utils.py:100-146):
    output word ``(k, z, c)`` (column ``z*(N/16)+c``) gathers input words
    ``4c..4c+3`` (bytes ``U[k, 16c .. 16c+15]``); slot ``i`` of every byte
    ``beta`` receives the 2-bit digit ``z`` (MSB first) of ``U[k, 16c+4i+beta]``
    at bits ``8*beta + 6 - 2i``.
    """
    U = np.ascontiguousarray(U, dtype=np.uint8)
    K, N = U.shape
    assert N % 16 == 0
    Z = max_bits // 2
    A = U.view("<u4").reshape(K, N // 16, 4).astype(np.uint32)  # [K, c, i]
    out = np.zeros((K, Z, N // 16), dtype=np.uint32)
    for z in range(Z):
        src = np.uint32((3 - z) * 2)
        acc = np.zeros((K, N // 16), dtype=np.uint32)
        for i in range(4):
            dst = np.uint32((3 - i) * 2)
            acc |= ((A[:, :, i] >> src) & np.uint32(0x03030303)) << dst
        out[:, z, :] = acc
    return out.reshape(K, Z * (N // 16))


def unpack_planes(B: np.ndarray, rows, bit_level: int, original_n: int) -> np.ndarray:
    """S5. ``unpack_pyt`` (grinqh/utils.py:149-177) for the uint32 layout.

    ``bit_level`` is the plane count ``Z`` (``BitLevel.value``).  Returns uint32
    ``[len(rows), original_n]`` whose bytes are the unsigned ``b``-bit codes
    ``U >> (8-b)`` in preshuffled column order.
    """
    k = int(bit_level)
    n_zone = original_n // 4
    if isinstance(rows, (int, np.integer)):
        rows = np.array([rows])
    rows = np.asarray(rows)
    pz = B.view(np.uint32)[rows, : n_zone * k].reshape(len(rows), k, n_zone)
    res = np.zeros((len(rows), n_zone, 4), dtype=np.uint32)
    for z in range(k):
        merge = np.uint32(2 * (k - 1 - z))
        for j, s in enumerate((6, 4, 2, 0)):
            res[:, :, j] += ((pz[:, z, :] >> np.uint32(s)) & np.uint32(0x03030303)) << merge
    return res.reshape(len(rows), n_zone * 4)


def prepare_weight(w_int8: np.ndarray, max_bits: int) -> np.ndarray:
    """``process_weights_after_loading`` data path (grinqh/grinqh.py:200-210):
    preshuffle -> shift -> plane pack."""
    return pack_planes(shift_codes(preshuffle(w_int8), max_bits), max_bits)


def decode_weight(B: np.ndarray, max_bits: int, original_n: int) -> np.ndarray:
    """F1's unpack + sign extend + postshuffle (grinqh/kernel.py:568-576) -> int8 ``W``."""
    K = B.shape[0]
    codes = unpack_planes(B, np.arange(K), max_bits // 2, original_n).view(np.uint8)
    sh = 8 - max_bits
    signed = ((codes.astype(np.int16) << sh).astype(np.uint8).view(np.int8).astype(np.int16) >> sh).astype(np.int8)
    return postshuffle(signed)


# ----------------------------------------------------------------------------
# S6 / S7 : grading and effective integer weights
# ----------------------------------------------------------------------------

def to_f32_threshold(thresholds) -> np.ndarray:
    """Thresholds as the Triton kernel sees them: python doubles rounded RNE to
    fp32 (triton/language/core.py tensor.__gt__ -> semantic.py promotion), padded
    / truncated to 4 like ``get_quant_method`` (grinqh/grinqh.py:111)."""
    t = list(thresholds) + [0.0] * 4
    return np.array(t[:4], dtype=np.float64).astype(np.float32)


def grade(sigma: np.ndarray, thresholds, max_bits: int) -> np.ndarray:
    """S6. Per-row zone bits: bit ``z`` set iff ``z < Z`` and
    ``fp32(|sigma|) > fp32(t_z)`` (grinqh/kernel.py:100-106, 116-118;
    tests/test_grinqh_ops.py:37, 45-47).  NaN compares false."""
    t = to_f32_threshold(thresholds)
    a = np.abs(np.asarray(sigma).astype(np.float32))
    Z = max_bits // 2
    bits = np.zeros(a.shape, dtype=np.uint8)
    with np.errstate(invalid="ignore"):
        for z in range(Z):
            bits |= (a > t[z]).astype(np.uint8) << np.uint8(z)
    return bits


def zone_mask_byte(zone_bits: np.ndarray) -> np.ndarray:
    """Byte mask ``OR_z act_z * (0xC0 >> 2z)`` (tests/test_grinqh_ops.py:47)."""
    m = np.zeros(zone_bits.shape, dtype=np.uint8)
    for z in range(4):
        m |= np.where((zone_bits >> z) & 1, np.uint8(0xC0 >> (2 * z)), np.uint8(0))
    return m


def midpoint_bias(zone_bits: np.ndarray, max_bits: int) -> np.ndarray:
    """S7 telescoped midpoint bias ``beta = sum_{z active} Delta_z`` with
    ``Delta_0 = B>>2``, ``Delta_z = (B>>(2z+2)) - (B>>2z)``, ``B = 1 << (b-1)``
    (grinqh/kernel.py:73-82, 108-113; tests/test_grinqh_ops.py:42-51)."""
    base = 1 << (max_bits - 1)
    beta = np.zeros(zone_bits.shape, dtype=np.int32)
    prev = 0
    for z in range(max_bits // 2):
        cur = base >> (2 * z + 2)
        beta += ((zone_bits >> z) & 1).astype(np.int32) * (cur - prev)
        prev = cur
    return beta


def effective_weight(w_int8: np.ndarray, zone_bits: np.ndarray, max_bits: int) -> np.ndarray:
    """S7. ``w_eff[k,n] = (int8(U[k,n] & mask_k) >> sh) + beta_k`` as int32
    (grinqh/kernel.py:116-146; tests/test_grinqh_ops.py:38-55)."""
    sh = 8 - max_bits
    U = shift_codes(w_int8, max_bits)
    mask = zone_mask_byte(zone_bits)
    masked = (U & mask[:, None]).view(np.int8).astype(np.int32) >> sh
    return masked + midpoint_bias(zone_bits, max_bits)[:, None]


def masked_weight_ref(w_int8: np.ndarray, x_row: np.ndarray, thresholds, max_bits: int) -> np.ndarray:
    """``get_masked_weight_ref`` (tests/test_grinqh_ops.py:28-55) in float64."""
    bits = grade(np.asarray(x_row).reshape(-1), thresholds, max_bits)
    return effective_weight(w_int8, bits, max_bits).astype(np.float64)


# ----------------------------------------------------------------------------
# S8 / S9 / S10 / S11 : products
# ----------------------------------------------------------------------------

def rne_cast(y: np.ndarray, dtype: str) -> np.ndarray:
    """Round-to-nearest-even cast of float64/float32 values to fp16 or bf16,
    returned as float64 for comparison."""
    y32 = np.asarray(y, dtype=np.float64).astype(np.float32)
    if dtype == "float16":
        return y32.astype(np.float16).astype(np.float64)
    if dtype == "bfloat16":
        u = y32.view(np.uint32).astype(np.uint64)
        nan = np.isnan(y32)
        rnd = ((u >> 16) & 1) + 0x7FFF
        r = ((u + rnd) >> 16) << 16
        out = r.astype(np.uint32).view(np.float32).astype(np.float64)
        out[nan] = np.nan
        return out
    raise ValueError(dtype)


def bias_add(y16: np.ndarray, bias, dtype: str) -> np.ndarray:
    """``y.to(dtype)`` followed by ``y.add_(bias)`` in the activation dtype
    (grinqh/kernel.py:706-708): two roundings."""
    y = rne_cast(y16, dtype)
    if bias is None:
        return y
    return rne_cast(y + np.asarray(bias, dtype=np.float64)[None, :], dtype)


def _scale_rows(scale: np.ndarray, K: int, group_size: int) -> np.ndarray:
    return np.repeat(np.asarray(scale, dtype=np.float64), group_size, axis=0)[:K]


def gemv_f64(x: np.ndarray, w_int8: np.ndarray, scale: np.ndarray, thresholds, max_bits: int,
             group_size: int) -> np.ndarray:
    """S8 in float64 before the output cast: ``y[n] = sum_k x_k * w_eff[k,n] *
    scale[k//gs, n]`` (grinqh/kernel.py:91-158).  ``x`` is ``[1, K]``."""
    x = np.asarray(x, dtype=np.float64).reshape(1, -1)
    K = x.shape[1]
    bits = grade(x[0], thresholds, max_bits)
    weff = effective_weight(w_int8, bits, max_bits).astype(np.float64)
    return x @ (weff * _scale_rows(scale, K, group_size))


def gemv(x, w_int8, scale, bias, thresholds, max_bits, group_size, dtype="float16"):
    """S8 with the fp16/bf16 output cast and bias add (grinqh/kernel.py:681-708)."""
    return bias_add(gemv_f64(x, w_int8, scale, thresholds, max_bits, group_size), bias, dtype)


def union_sigma(x: np.ndarray) -> np.ndarray:
    """Statistic of the batch-union grading, ``sigma_k = max_m |x[m,k]|``
    (grinqh/kernel.py:237-249).  The kernel holds the batch in one tile of
    ``BLOCK_BATCH = next_power_of_2(M)`` rows (:196-197, :632) whose rows past
    ``M`` load as 0.0 (``other=0.0``, :240-245), and reduces ``|x|`` with
    ``tl.max``, which combines pairs with ``tl.maximum`` at its default
    ``propagate_nan=NONE`` -- a NaN-ignoring maximum (maxnum).  So NaN entries
    are ignored, and a column whose entries are all NaN has statistic NaN
    when ``M`` is a power of two and 0.0 (the padding rows) otherwise."""
    x = np.asarray(x, dtype=np.float64)
    sigma = np.fmax.reduce(np.abs(x), axis=0)
    M = x.shape[0]
    if M & (M - 1):
        sigma = np.fmax(sigma, 0.0)
    return sigma


def gemv_union_f64(x: np.ndarray, w_int8: np.ndarray, scale: np.ndarray, thresholds, max_bits: int,
                   group_size: int) -> np.ndarray:
    """S10: grade row ``k`` on ``sigma_k = max_m |x[m,k]|`` (``union_sigma``,
    grinqh/kernel.py:249-289), then ``y[m,n] = sum_k x[m,k] w_eff[k,n]
    scale[k//gs,n]`` (:339-344)."""
    x = np.asarray(x, dtype=np.float64)
    K = x.shape[1]
    sigma = union_sigma(x)
    bits = grade(sigma, thresholds, max_bits)
    weff = effective_weight(w_int8, bits, max_bits).astype(np.float64)
    return x @ (weff * _scale_rows(scale, K, group_size))


def gemv_union(x, w_int8, scale, bias, thresholds, max_bits, group_size, dtype="float16"):
    """S10 with output cast and bias (grinqh/kernel.py:639-643)."""
    return bias_add(gemv_union_f64(x, w_int8, scale, thresholds, max_bits, group_size), bias, dtype)


def dense_weight(w_int8: np.ndarray, scale: np.ndarray, group_size: int, dtype: str) -> np.ndarray:
    """S9 elementwise: ``Wd = RNE_dtype(W * scale[k//gs])`` (grinqh/kernel.py:578-586)."""
    K = w_int8.shape[0]
    s = rne_cast(_scale_rows(scale, K, group_size), dtype)
    return rne_cast(w_int8.astype(np.float64) * s, dtype)


def graded_weight_rounded(w_int8: np.ndarray, zone_bits: np.ndarray, scale: np.ndarray, max_bits: int,
                          group_size: int, dtype: str) -> np.ndarray:
    """``RNE_dtype(w_eff[k,n] * scale[k//gs,n])``: the S7 effective weight scaled
    and rounded once to the activation dtype, the way S9 rounds the dense weight
    (grinqh/kernel.py:578-586).  With every zone active it is ``dense_weight``.
    This is the weight a graded kernel multiplies when it applies the scale
    before the matmul instead of after it (the reference's S10 keeps
    ``x * w_eff`` and the scale in fp32, grinqh/kernel.py:321-344)."""
    K = w_int8.shape[0]
    weff = effective_weight(w_int8, zone_bits, max_bits).astype(np.float64)
    s = rne_cast(_scale_rows(scale, K, group_size), dtype)
    with np.errstate(over="ignore"):
        return rne_cast(weff * s, dtype)


def gemv_union_rounded_f64(x: np.ndarray, w_int8: np.ndarray, scale: np.ndarray, thresholds, max_bits: int,
                           group_size: int, dtype: str) -> np.ndarray:
    """S10 with the scaled effective weight rounded to the activation dtype
    before the product: ``x @ graded_weight_rounded(...)`` in float64, grading
    on the union statistic (grinqh/kernel.py:249-289)."""
    x = np.asarray(x, dtype=np.float64)
    sigma = union_sigma(x)
    bits = grade(sigma, thresholds, max_bits)
    return x @ graded_weight_rounded(w_int8, bits, scale, max_bits, group_size, dtype)


def dense_exact_f64(x, w_int8, scale, group_size) -> np.ndarray:
    """Dense product with the scale kept exact (``x @ (W * s)`` in float64, no
    rounding of ``W*s``): S10 with every zone active (tests/test_grinqh_ops.py:170,
    190), what a kernel that applies the scale in fp32 computes for the
    dense dispatch."""
    x = np.asarray(x, dtype=np.float64)
    return x @ (w_int8.astype(np.float64) * _scale_rows(scale, w_int8.shape[0], group_size))


def dense_prefill_f64(x, w_int8, scale, group_size, dtype="float16") -> np.ndarray:
    """S9 product in float64 before the output cast: ``X @ Wd`` (grinqh/kernel.py:587)."""
    return np.asarray(x, dtype=np.float64) @ dense_weight(w_int8, scale, group_size, dtype)


def dense_prefill(x, w_int8, scale, bias, group_size, dtype="float16"):
    """S9 with output cast and bias (grinqh/kernel.py:561-587, 707-708)."""
    return bias_add(dense_prefill_f64(x, w_int8, scale, group_size, dtype), bias, dtype)


def gemm_or_gemv(x, w_int8, scale, bias, max_bits, group_size, thresholds, dtype="float16",
                 batch_grading="reference"):
    """S11 dispatch (grinqh/kernel.py:646-710): one row -> graded GEMV; more
    rows -> dense dequantize-then-matmul.  ``batch_grading="union"`` grades every
    batch with the S10 union rule instead."""
    x2 = np.asarray(x, dtype=np.float64).reshape(-1, np.shape(x)[-1])
    if batch_grading == "union":
        y = gemv_union(x2, w_int8, scale, bias, thresholds, max_bits, group_size, dtype)
    elif x2.shape[0] > 1:
        y = dense_prefill(x2, w_int8, scale, bias, group_size, dtype)
    else:
        y = gemv(x2, w_int8, scale, bias, thresholds, max_bits, group_size, dtype)
    return y.reshape(tuple(np.shape(x)[:-1]) + (w_int8.shape[1],))
