"""The allocation-free entry point grinqh_gemm_or_gemv_noalloc (include/grinqh.h)
against the workspace entry point grinqh_gemm_or_gemv, through the C ABI.

Each case calls the allocation-free entry point twice in a row, the second
time with a smaller batch (the scratch array keeps the first call's contents:
counters must be back at zero, partial sums must not leak), and checks both
results bitwise against grinqh_gemm_or_gemv on the same inputs: the GEMV
(one and four rows), the decode kernel (graded and dense), the fused prefill
(graded, dense, and split over K).  Where the workspace entry point takes
the library GEMM the allocation-free one runs the hand-written large-batch
kernel, and where a decode launch's split-K partial sums outgrow the fixed
scratch it runs the rows in chunks: those cases are held to the oracle
instead.
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


def test_noalloc_large_batch_without_library(lib):
    """512 rows: the allocation-free entry point runs the hand-written
    large-batch kernel (no dense weight buffer); it computes S9 (RNE(w*s), the
    dense dispatch) and is held to the oracle."""
    from grinqh.utils import prepare_weight
    rng = np.random.default_rng(3)
    M, K, N = 512, 1024, 2048
    W, x, s, b = _inputs(rng, M, K, N)
    P = prepare_weight(torch.from_numpy(W).cuda(), 8)
    y = _noalloc(lib, _dev(x), P, _dev(s), _dev(b), N, [0.0] * 4, "dense")
    pre = O.dense_prefill_f64(x, W, s, 128, "float16")
    assert_output_close(y, pre, O.dense_prefill(x, W, s, b, 128, "float16"), "float16", bias=b,
                        what="noalloc 512-row prefill")


@pytest.mark.parametrize("M", [40, 64])
def test_noalloc_large_k_decode_runs_in_row_chunks(lib, M):
    """Llama-3-405B down_proj (K = 53248, N = 16384): a decode launch of M
    rows needs at least 26 K ranges of M x N fp32 partial sums (68 MiB at 40
    rows, 104 MiB at 64), more than the 64 MiB scratch.  The allocation-free
    entry point then runs the rows in chunks that fit, graded on the whole
    batch's statistic (reduced once into the scratch), and the result is held
    to the oracle (32-row chunks, like 40 and 64 rows, take the rounded scaled
    weight) on a slice of the columns, twice in a row; a following small call
    shows the counters are back at zero."""
    from grinqh.utils import prepare_weight
    K, N = 53248, 16384
    rng = np.random.default_rng(405)
    W = rng.integers(-128, 128, size=(K, N), dtype=np.int8)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    s = to_dtype_np(rng.standard_normal((K // 128, N)) * 0.02, "float16")
    P = prepare_weight(torch.from_numpy(W).cuda(), 8)
    st = _dev(s)
    sigma = np.abs(x).max(0).astype(np.float32)
    t = [0.0] + np.quantile(sigma, [0.5, 0.8, 0.95]).tolist()
    cols = np.r_[0:256, N - 256:N]
    pre = O.gemv_union_rounded_f64(x, W[:, cols], s[:, cols], t, 8, 128, "float16")
    fin = O.bias_add(pre, None, "float16")
    xt = _dev(x)
    for _ in range(2):
        y = _noalloc(lib, xt, P, st, None, N, t, "union")
        assert_output_close(y[:, torch.from_numpy(cols).cuda()], pre, fin, "float16",
                            what=f"noalloc 405B down_proj M={M}")
    # a small call after: the split-K counters the chunks used are zero again
    xs = _dev(x[:4])
    pre4 = O.gemv_union_f64(x[:4], W[:, cols], s[:, cols], t, 8, 128)
    y4 = _noalloc(lib, xs, P, st, None, N, t, "union")
    assert_output_close(y4[:, torch.from_numpy(cols).cuda()], pre4, O.bias_add(pre4, None, "float16"), "float16",
                        what="noalloc 405B down_proj M=4 after the chunked call")
