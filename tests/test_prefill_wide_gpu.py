"""The wide-tile fp16 prefill kernel (256 x 256 output tiles, the weight
dequantized into LDS), through the C ABI.

It serves fp16 batches of 512 rows and more whose tile grid fills the GPU
(N % 256 == 0, at least 192 tiles of 256 x 256) when the product may not
allocate the dense weight: the allocation-free entry point
grinqh_gemm_or_gemv_noalloc.  It computes the reference's dense dispatch S9
(grinqh/kernel.py:561-587: x @ RNE(W * s), fp32 accumulation, bias added in
the activation dtype) and, graded, x @ RNE(w_eff * s), so it is held to the
oracle variants that round the scaled weight the same way, at the base
tolerance (no weight-rounding allowance).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import assert_output_close, error_stats, rand_weight, record_errors, to_dtype_np

pytestmark = pytest.mark.gpu

BITS = [2, 4, 6, 8]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from grinqh import _lib
    return _lib.load_library()


def _dev(a):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(torch.float16).cuda()


def _weights(rng, K, N, b, scale_sd=0.02):
    from grinqh.utils import prepare_weight
    W = rand_weight(rng, K, N, b)
    s = to_dtype_np(rng.standard_normal((-(-K // 128), N)) * scale_sd, "float16")
    return W, s, prepare_weight(torch.from_numpy(W).cuda(), b)


def _noalloc(lib, xt, P, st, bt, N, b, t, mode):
    from grinqh import _lib
    M, K = xt.shape
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    rc = lib.grinqh_gemm_or_gemv_noalloc(
        xt.data_ptr(), M, K, xt.stride(0), N, _lib.DTYPE_F16, P.data_ptr(), st.data_ptr(),
        bt.data_ptr() if bt is not None else None, y.data_ptr(), b, 128, _lib.thresholds_f32(t),
        {"union": _lib.MODE_UNION, "dense": _lib.MODE_DENSE}[mode], ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "grinqh_gemm_or_gemv_noalloc")
    return y


def _round_significand(v, bits=11):
    """RNE to `bits` significant bits with no exponent limit (fp16 precision
    without fp16's range)."""
    m, e = np.frexp(np.asarray(v, dtype=np.float64))
    return np.ldexp(np.round(m * 2.0 ** bits) / 2.0 ** bits, e)


@pytest.mark.parametrize("max_bits", BITS)
def test_wide_prefill_dense(lib, max_bits):
    """Dense (S9) at 520 rows (three row blocks, the last one 8 rows deep),
    K = 512 (eight 64-row stages, scale groups of two), N = 16384 (192
    tiles), with bias: x @ RNE(W * s), rounded, plus bias."""
    rng = np.random.default_rng(5100 + max_bits)
    M, K, N = 520, 512, 16384
    W, s, P = _weights(rng, K, N, max_bits)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    bias = to_dtype_np(rng.standard_normal(N), "float16")
    y = _noalloc(lib, _dev(x), P, _dev(s), _dev(bias), N, max_bits, [0.0] * 4, "dense")
    pre = O.dense_prefill_f64(x, W, s, 128, "float16")
    fin = O.dense_prefill(x, W, s, bias, 128, "float16")
    assert_output_close(y, pre, fin, "float16", bias=bias, what=f"wide prefill dense b={max_bits}")
    record_errors("wide prefill, allocation-free entry point (K=512, N=16384, bias)", f"M={M} dense b={max_bits}",
                  rows_checked=M, weight_rounded=True, vs_reference=error_stats(y, fin), vs_own=error_stats(y, fin))


@pytest.mark.parametrize("group_size", [64, 256])
def test_wide_prefill_group_sizes(lib, group_size):
    """Scale groups of 64 rows (a new group every 64-row stage) and of 256
    rows (one group over four stages), dense, K = 1024, 512 rows, bias."""
    from grinqh.utils import prepare_weight
    rng = np.random.default_rng(5700 + group_size)
    M, K, N, b = 512, 1024, 24576, 8
    W = rand_weight(rng, K, N, b)
    s = to_dtype_np(rng.standard_normal((K // group_size, N)) * 0.02, "float16")
    P = prepare_weight(torch.from_numpy(W).cuda(), b)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    bias = to_dtype_np(rng.standard_normal(N), "float16")
    from grinqh import _lib
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    xt, st, bt = _dev(x), _dev(s), _dev(bias)
    rc = lib.grinqh_gemm_or_gemv_noalloc(
        xt.data_ptr(), M, K, xt.stride(0), N, _lib.DTYPE_F16, P.data_ptr(), st.data_ptr(), bt.data_ptr(),
        y.data_ptr(), b, group_size, _lib.thresholds_f32([0.0] * 4), _lib.MODE_DENSE,
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "grinqh_gemm_or_gemv_noalloc")
    pre = O.dense_prefill_f64(x, W, s, group_size, "float16")
    fin = O.dense_prefill(x, W, s, bias, group_size, "float16")
    assert_output_close(y, pre, fin, "float16", bias=bias, what=f"wide prefill group size {group_size}")


@pytest.mark.parametrize("max_bits", [4, 8])
@pytest.mark.parametrize("t", [[0.5, 0.1, 2.0, 1.0], [float("inf")] * 4, [-1.0] * 4, [0.0, 0.2, 0.2, 3.0], None],
                         ids=["non_monotone", "skip_all", "all_planes", "tied", "quantiles"])
def test_wide_prefill_graded(lib, t, max_bits):
    """Union grading at 512 rows, K = 1024, N = 24576 (192 tiles), with bias:
    each row of K takes the zone set of sigma_k = max_m |x[m][k]|, inactive
    planes masked to zero and the midpoint bias added, the weight rounded as
    RNE(w_eff * s).  Zone sets that are not prefixes, none, all, tied
    thresholds and the 70/20/8/2 % quantile mix."""
    rng = np.random.default_rng(5200 + max_bits)
    M, K, N = 512, 1024, 24576
    W, s, P = _weights(rng, K, N, max_bits)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    if t is None:
        sigma = O.union_sigma(x)
        t = [0.0] + np.quantile(sigma, [0.7, 0.9, 0.98]).tolist()
    bias = to_dtype_np(rng.standard_normal(N), "float16")
    y = _noalloc(lib, _dev(x), P, _dev(s), _dev(bias), N, max_bits, t, "union")
    pre = O.gemv_union_rounded_f64(x, W, s, t, max_bits, 128, "float16")
    fin = O.bias_add(pre, bias, "float16")
    assert_output_close(y, pre, fin, "float16", bias=bias, what=f"wide prefill graded t={t}")


def test_wide_prefill_strided_rows(lib):
    """Activation rows with a leading dimension above K (a column slice of a
    wider tensor), 600 rows, K = 384, no bias, twice in a row."""
    rng = np.random.default_rng(5300)
    M, K, N, b = 600, 384, 16384, 8
    W, s, P = _weights(rng, K, N, b)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    wide = np.concatenate([x, to_dtype_np(rng.standard_normal((M, 64)), "float16")], axis=1)
    xt = _dev(wide)[:, :K]
    assert xt.stride(0) == K + 64
    pre = O.dense_prefill_f64(x, W, s, 128, "float16")
    fin = O.dense_prefill(x, W, s, None, 128, "float16")
    for _ in range(2):
        y = _noalloc(lib, xt, P, _dev(s), None, N, b, [0.0] * 4, "dense")
        assert_output_close(y, pre, fin, "float16", what="wide prefill, strided rows")


def test_wide_prefill_gate_up_shape(lib):
    """Llama-3-8B gate_up (K = 4096, N = 28672) at 600 rows, dense and graded
    (70/20/8/2 % mix): the first 64 rows and the partial last row block are
    held to the oracle."""
    rng = np.random.default_rng(5400)
    M, K, N, b = 600, 4096, 28672, 8
    W, s, P = _weights(rng, K, N, b)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    rows = np.r_[0:64, 512:600]
    sigma = O.union_sigma(x)
    t = [0.0] + np.quantile(sigma, [0.7, 0.9, 0.98]).tolist()
    for mode in ("dense", "union"):
        y = _noalloc(lib, _dev(x), P, _dev(s), None, N, b, t if mode == "union" else [0.0] * 4, mode)
        ys = y[torch.from_numpy(rows).cuda()]
        if mode == "dense":
            pre = O.dense_prefill_f64(x[rows], W, s, 128, "float16")
            fin = O.dense_prefill(x[rows], W, s, None, 128, "float16")
        else:  # the zone sets come from the whole batch's statistic
            weff = O.effective_weight(W, O.grade(sigma, t, b), b).astype(np.float64)
            wd = (weff * np.repeat(s.astype(np.float64), 128, axis=0)).astype(np.float16).astype(np.float64)
            pre = x[rows].astype(np.float64) @ wd
            fin = O.bias_add(pre, None, "float16")
        assert_output_close(ys, pre, fin, "float16", what=f"wide prefill gate_up {mode}")
        record_errors("wide prefill, allocation-free entry point: Llama-3-8B gate_up", f"M={M} {mode}",
                      rows_checked=len(rows), weight_rounded=True, vs_reference=error_stats(ys, fin),
                      vs_own=error_stats(ys, fin))


def test_wide_prefill_scales_beyond_the_fp16_weight_range(lib):
    """fp16 scales of 600-1500 (|w_eff * s| up to ~1.9e5, past 65504), graded:
    a block whose scales reach past 65504 / 2^(max_bits-1) builds the weight
    from s * 2^-e and scales its sums by 2^e, so the result is x @ R(w_eff * s)
    with R fp16's 11-bit rounding without its range limit, finite."""
    rng = np.random.default_rng(5500)
    M, K, N, b = 520, 512, 16384, 8
    W = rand_weight(rng, K, N, b)
    from grinqh.utils import prepare_weight
    P = prepare_weight(torch.from_numpy(W).cuda(), b)
    x = to_dtype_np(rng.standard_normal((M, K)) * 1e-4, "float16")
    s = to_dtype_np(np.where(rng.random((K // 128, N)) < 0.5, -1.0, 1.0) * rng.uniform(600, 1500, (K // 128, N)),
                    "float16")
    bias = to_dtype_np(rng.standard_normal(N), "float16")
    sigma = O.union_sigma(x)
    t = [0.0] + np.quantile(sigma, [0.5, 0.8, 0.95]).tolist()
    y = _noalloc(lib, _dev(x), P, _dev(s), _dev(bias), N, b, t, "union")
    weff = O.effective_weight(W, O.grade(sigma, t, b), b).astype(np.float64)
    pre = x.astype(np.float64) @ _round_significand(weff * np.repeat(s.astype(np.float64), 128, axis=0))
    fin = O.bias_add(pre, bias, "float16")
    assert np.isfinite(fin).all()
    assert_output_close(y, pre, fin, "float16", bias=bias, what="wide prefill, scales past the fp16 weight range")


def test_wide_prefill_nonfinite_rows(lib):
    """A NaN or inf activation makes its whole output row NaN (graded), as the
    reference's sum of beta * x does (grinqh/kernel.py:113-114); the other
    rows stay finite."""
    rng = np.random.default_rng(5600)
    M, K, N, b = 520, 256, 16384, 8
    W, s, P = _weights(rng, K, N, b)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16").copy()
    x[0, 17] = np.nan
    x[M - 1, 200] = np.inf
    y = _noalloc(lib, _dev(x), P, _dev(s), None, N, b, [0.1, 0.5, 1.0, 2.0], "union").float().cpu()
    assert torch.isnan(y[0]).all() and torch.isnan(y[M - 1]).all()
    assert torch.isfinite(y[1:M - 1]).all()
