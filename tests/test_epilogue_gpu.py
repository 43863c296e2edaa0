"""Bit-exact check of the output epilogue on every product path.

The reference casts the fp32 (one row) or matmul (more rows) result to the
activation dtype and then adds the bias in that dtype: two roundings
(grinqh/kernel.py:697-708).  Rounding ``acc + bias`` once differs from that in
the last bit for some outputs, which a tolerance of a few units of roundoff
cannot see.  Here the operands are small integers, the codes are 8-bit and the
scales powers of two, so every product and every partial sum is exact in fp32
whatever the summation order, and the only roundings left are the epilogue's.
Each path -- the graded GEMV (1 row), the four-row GEMV, the decode kernels
(5-64 rows), the fused prefill (65-255), the library-GEMM prefill and the
hand-written large-batch prefill (256 rows and more, with and without a
workspace) -- must then equal the oracle's cast-then-add bit for bit, in
fp16 and bf16, dense and graded.  The test also counts the outputs where one
rounding would have given another value, so it cannot pass vacuously.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import TORCH_DTYPES

pytestmark = pytest.mark.gpu

B = 8
# union thresholds on sigma in {0, 1, 2}: no zone, zone 0 only, zones 0-2
T_UNION = [0.5, 1.5, 1.5, 2.5]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from grinqh import _lib
    return _lib.load_library()


def _operands(seed, M, K, N):
    rng = np.random.default_rng(seed)
    lim = 1 << (B - 1)
    W = rng.integers(-lim, lim, size=(K, N)).astype(np.int8)
    x = rng.integers(-2, 3, size=(M, K)).astype(np.float64)
    s = rng.choice([0.25, 0.5, 1.0], size=(K // 128, N)).astype(np.float64)
    bias = rng.integers(-6, 7, size=N).astype(np.float64)
    return W, x, s, bias


def _expected(x, W, s, bias, mode, dtype):
    """The exact product (every term and sum is exact), then the oracle's
    epilogue; also the number of outputs where one rounding of acc + bias
    would differ."""
    M = x.shape[0]
    if mode == "union" or (mode == "reference" and M == 1):
        pre = O.gemv_union_f64(x, W, s, T_UNION, B, 128)
    else:
        pre = O.dense_exact_f64(x, W, s, 128)
    # the dense weight W * s is exact in both dtypes here, so S9 is this product too
    assert np.array_equal(pre, O.dense_prefill_f64(x, W, s, 128, dtype)) or mode != "dense"
    want = O.bias_add(pre, bias, dtype)
    once = O.rne_cast(pre + bias[None, :], dtype)
    return want, int((once != want).sum())


def _dev(a, dtype):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(TORCH_DTYPES[dtype]).cuda()


def _prepare(W):
    from grinqh.utils import prepare_weight
    return prepare_weight(torch.from_numpy(W).cuda(), B)


def _noalloc(lib, xt, P, st, bt, N, mode, dtype):
    from grinqh import _lib
    M, K = xt.shape
    y = torch.empty((M, N), dtype=xt.dtype, device="cuda")
    rc = lib.grinqh_gemm_or_gemv_noalloc(
        xt.data_ptr(), M, K, xt.stride(0), N, _lib.DTYPE_F16 if dtype == "float16" else _lib.DTYPE_BF16,
        P.data_ptr(), st.data_ptr(), bt.data_ptr(), y.data_ptr(), B, 128, _lib.thresholds_f32(T_UNION),
        {"reference": _lib.MODE_REFERENCE, "union": _lib.MODE_UNION, "dense": _lib.MODE_DENSE}[mode],
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "grinqh_gemm_or_gemv_noalloc")
    return y


# (rows, K, N, mode, entry point): one case per kernel the dispatch can take
CASES = [
    (1, 512, 1024, "reference", "op"),     # graded one-row GEMV
    (1, 512, 1024, "dense", "op"),         # dense one-row GEMV
    (3, 512, 1024, "union", "op"),         # four-row GEMV
    (16, 512, 1024, "union", "op"),        # decode kernel, one m-tile
    (40, 512, 1024, "dense", "op"),        # decode kernel, rounded-weight path in fp16
    (64, 1024, 2048, "union", "op"),       # decode kernel, four m-tiles
    (100, 512, 1024, "dense", "op"),       # fused prefill
    (200, 512, 1024, "union", "op"),       # graded fused prefill
    (512, 512, 1024, "dense", "op"),       # library GEMM prefill (the default for this shape)
    (600, 256, 2048, "union", "op"),       # graded library GEMM prefill
    (512, 512, 1024, "dense", "tall"),     # hand-written large-batch kernel, with a workspace
    (600, 256, 2048, "union", "tall"),
    (2048, 256, 6144, "dense", "noalloc"),  # large-batch kernel without a workspace
    (2048, 256, 6144, "union", "noalloc"),
]


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("M,K,N,mode,entry", CASES,
                         ids=[f"{c[3]}-M{c[0]}-{c[4]}" for c in CASES])
def test_epilogue_is_cast_then_add_bit_exact(lib, M, K, N, mode, entry, dtype, monkeypatch):
    from grinqh import _lib
    from grinqh.kernel import run_product
    dt = _lib.DTYPE_F16 if dtype == "float16" else _lib.DTYPE_BF16
    mc = {"reference": _lib.MODE_REFERENCE, "union": _lib.MODE_UNION, "dense": _lib.MODE_DENSE}[mode]
    if entry == "tall":
        monkeypatch.setenv("GRINQH_PREFILL", "tall")
    if M >= 512:  # the case reaches the kernel it names
        want_kernel = _lib.KERNEL_LIBRARY if entry == "op" else _lib.KERNEL_TALL
        assert _lib.product_kernel(M, K, K, N, dt, B, 128, mc, entry == "noalloc")[0] == want_kernel
    W, x, s, bias = _operands(M * 31 + N + K, M, K, N)
    want, n_differ = _expected(x, W, s, bias, mode, dtype)
    assert n_differ > 0, "operands put no output where one rounding differs from two"
    xt, st, bt = _dev(x, dtype), _dev(s, dtype), _dev(bias, dtype)
    P = _prepare(W)
    if entry == "noalloc":
        y = _noalloc(lib, xt, P, st, bt, N, mode, dtype)
    else:
        y = run_product(xt, P, st, bt, B, 128, N // 4, T_UNION, mode)
    got = y.double().cpu().numpy()
    bad = got != want
    assert not bad.any(), (f"{int(bad.sum())} of {bad.size} outputs differ from cast-then-add "
                           f"({n_differ} outputs would differ under one rounding); first at "
                           f"{np.argwhere(bad)[0].tolist()}: got {got[bad][0]}, want {want[bad][0]}")
