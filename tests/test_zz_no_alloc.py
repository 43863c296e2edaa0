"""The allocation-free entry point grinqh_gemm_or_gemv_noalloc (include/grinqh.h)
against the workspace entry point grinqh_gemm_or_gemv, through the C ABI.

Each case calls the allocation-free entry point twice in a row, the second
time with a smaller batch (the scratch array keeps the first call's contents:
counters must be back at zero, partial sums must not leak), and checks both
results bitwise against grinqh_gemm_or_gemv on the same inputs: the GEMV
(one and four rows), the decode kernel (graded and dense), the fused prefill
(graded, dense, and split over K).  From 512 rows (and from 257 with
K <= 8192) the workspace entry point takes the library GEMM while the
allocation-free one keeps the fused kernels, so that case is held to the
oracle instead.
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import assert_output_close, rand_weight, to_dtype_np

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from grinqh import _lib
    return _lib.load_library()


def _inputs(rng, M, K, N, bias=True):
    W = rand_weight(rng, K, N, 8)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    s = to_dtype_np(rng.standard_normal((-(-K // 128), N)) * 0.02, "float16")
    b = to_dtype_np(rng.standard_normal(N), "float16") if bias else None
    return W, x, s, b


def _dev(a, dt=torch.float16):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(dt).cuda()


def _noalloc(lib, xt, P, st, bt, N, t, mode):
    from grinqh import _lib
    M, K = xt.shape
    y = torch.empty((M, N), dtype=torch.float16, device="cuda")
    stream = torch.cuda.current_stream().cuda_stream
    rc = lib.grinqh_gemm_or_gemv_noalloc(
        xt.data_ptr(), M, K, xt.stride(0), N, _lib.DTYPE_F16, P.data_ptr(), st.data_ptr(),
        bt.data_ptr() if bt is not None else None, y.data_ptr(), 8, 128, _lib.thresholds_f32(t),
        {"reference": _lib.MODE_REFERENCE, "union": _lib.MODE_UNION, "dense": _lib.MODE_DENSE}[mode],
        ctypes.c_void_p(stream))
    _lib.check(rc, "grinqh_gemm_or_gemv_noalloc")
    return y


# (K, N, mode, first M, second M): two calls in a row, the second smaller
CASES = [
    (14336, 4096, "reference", 1, 1),     # graded GEMV, split-K reduce kernel
    (4096, 28672, "union", 4, 2),         # four-row GEMV, in-kernel split-K completion
    (4096, 6144, "union", 64, 20),        # decode, batch statistic, scaled path
    (4096, 4096, "dense", 16, 5),         # decode, one m-tile
    (1024, 2048, "dense", 250, 100),      # fused prefill
    (512, 1024, "union", 200, 80),        # graded fused prefill
    (2080, 256, "dense", 100, 70),        # fused prefill split over K (partial sums)
]


@pytest.mark.parametrize("K,N,mode,m1,m2", CASES)
def test_noalloc_matches_workspace_entry_point(lib, K, N, mode, m1, m2):
    from grinqh.kernel import run_product
    from grinqh.utils import prepare_weight
    rng = np.random.default_rng(K + N + m1)
    W, x, s, b = _inputs(rng, m1, K, N)
    P = prepare_weight(torch.from_numpy(W).cuda(), 8)
    st, bt = _dev(s), _dev(b)
    sigma = np.abs(x).max(0).astype(np.float32)
    t = [0.0] + np.quantile(sigma, [0.5, 0.8, 0.95]).tolist()
    for M in (m1, m2):
        xt = _dev(x[:M])
        got = _noalloc(lib, xt, P, st, bt, N, t, mode)
        want = run_product(xt, P, st, bt, 8, 128, N // 4, t, mode)
        torch.cuda.synchronize()
        assert torch.equal(got, want), f"M={M}: max |diff| {(got.float() - want.float()).abs().max().item()}"


def test_noalloc_large_batch_stays_on_fused_kernel(lib):
    """512 rows: the allocation-free entry point runs the fused prefill (no
    dense weight buffer); it computes S9 (RNE(w*s), the dense dispatch) and
    is held to the oracle."""
    from grinqh.utils import prepare_weight
    rng = np.random.default_rng(3)
    M, K, N = 512, 1024, 2048
    W, x, s, b = _inputs(rng, M, K, N)
    P = prepare_weight(torch.from_numpy(W).cuda(), 8)
    y = _noalloc(lib, _dev(x), P, _dev(s), _dev(b), N, [0.0] * 4, "dense")
    pre = O.dense_prefill_f64(x, W, s, 128, "float16")
    assert_output_close(y, pre, O.dense_prefill(x, W, s, b, 128, "float16"), "float16", bias=b,
                        what="noalloc 512-row prefill")
