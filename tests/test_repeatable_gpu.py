"""Every product path returns the same bits on every call with the same inputs.

The kernels' reductions run in fixed orders (split-K ranges summed in range
order, K sub-ranges through LDS in fixed order), so a result that changes from
call to call can only come from a race or from a hardware hazard: e.g. a load
that overwrites an accumulator register before an MFMA issued earlier has read
it, which with two waves sharing a SIMD's matrix pipe shows up as a few wrong
outputs in a different place on every call.  Each case compares repeated
calls with the first, bit for bit (the other tests hold results to the
oracle), on the GEMV (1-4 rows), decode (5-64), fused prefill, library-GEMM
and hand-written large-batch paths, dense and graded, fp16 and bf16.
"""
import numpy as np
import pytest
import torch

from tests._helpers import TORCH_DTYPES, rand_weight, to_dtype_np

pytestmark = pytest.mark.gpu

REPEATS = 8
SHAPES = [(4096, 6144), (4096, 28672), (14336, 4096)]
# 20 and 33: the 17-32- and 33-64-row decode kernels with rows past the batch,
# whose two waves per K sub-range share each x tile through LDS
ROWS = [1, 3, 16, 20, 33, 40, 64, 128]


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from grinqh import _lib
    return _lib.load_library()


def _case(K, N, M, dtype, seed):
    from grinqh.utils import prepare_weight
    rng = np.random.default_rng(seed)
    W = rand_weight(rng, K, N, 8)
    s = to_dtype_np(rng.standard_normal((K // 128, N)) * 0.02, dtype)
    x = to_dtype_np(rng.standard_normal((M, K)), dtype)
    td = TORCH_DTYPES[dtype]
    dev = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(td).cuda()
    return dev(x), prepare_weight(torch.from_numpy(W).cuda(), 8), dev(s)


def _repeat_equal(x, P, s, N, mode):
    from grinqh.kernel import run_product
    t = [0.0, 0.5, 1.5, 2.5] if mode == "union" else [0.0] * 4
    y0 = run_product(x, P, s, None, 8, 128, N // 4, t, mode)
    differing = sum(not torch.equal(run_product(x, P, s, None, 8, 128, N // 4, t, mode), y0)
                    for _ in range(REPEATS))
    return differing


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("K,N", SHAPES, ids=[f"K{k}-N{n}" for k, n in SHAPES])
@pytest.mark.parametrize("mode", ["dense", "union"])
def test_decode_and_gemv_paths_repeat_bitwise(lib, dtype, K, N, mode):
    for M in ROWS:
        x, P, s = _case(K, N, M, dtype, K + N + M)
        assert _repeat_equal(x, P, s, N, mode) == 0, f"M={M}: a call gave different bits"


@pytest.mark.parametrize("path", ["library", "tall"])
@pytest.mark.parametrize("mode", ["dense", "union"])
def test_prefill_paths_repeat_bitwise(lib, path, mode, monkeypatch):
    """512 and 2048 rows of gate_up (the hand-written kernel's split last round
    at 2048) and of down, each path forced."""
    from grinqh import _lib
    monkeypatch.setenv("GRINQH_PREFILL", path)
    want = _lib.KERNEL_LIBRARY if path == "library" else _lib.KERNEL_TALL
    for K, N in [(4096, 28672), (14336, 4096)]:
        for M in (512, 2048):
            mc = _lib.MODE_UNION if mode == "union" else _lib.MODE_DENSE
            assert _lib.product_kernel(M, K, K, N, _lib.DTYPE_F16, 8, 128, mc)[0] == want
            x, P, s = _case(K, N, M, "float16", K + N + M)
            assert _repeat_equal(x, P, s, N, mode) == 0, f"{path} K={K} N={N} M={M}: a call gave different bits"
