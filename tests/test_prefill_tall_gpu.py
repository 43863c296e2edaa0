"""The large-batch prefill kernel (prefill_tall_kernel: 512 x 128 or
256 x 128 output tiles over four waves, one per SIMD, x repacked into MFMA
fragments and loaded straight into registers, the weight dequantized once
per block and stage into LDS), through the C ABI.

It takes a prefill from kTallPrefillRows rows whose shape it fits (K and the
group size multiples of 64, N % 128 == 0): always without a workspace, with
one where the dispatch prefers it over the library path (up to 512 rows for
the larger weights) or where GRINQH_PREFILL=tall asks for it, as here.
It computes the reference's dense dispatch S9 (grinqh/kernel.py:561-587:
x @ RNE(W * s), fp32 accumulation, the bias added in the activation dtype)
and, graded, x @ RNE(w_eff * s) on the batch statistic, so it is held to the
oracle variants that round the scaled weight the same way, at the base
tolerance.  grinqh_product_kernel names the kernel and its plan, so every
test first checks that the case reaches the plan it is meant to cover
(one or several K ranges, 512- or 256-row blocks).
"""
import ctypes

import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import TORCH_DTYPES, assert_output_close, error_stats, rand_weight, record_errors, to_dtype_np

pytestmark = pytest.mark.gpu

BITS = [2, 4, 6, 8]
DTYPES = ["float16", "bfloat16"]


@pytest.fixture(autouse=True)
def _tall_path(monkeypatch):
    """Pin the large-batch kernel: by default the dispatch hands most of these
    shapes to the library path (dense weight + library GEMM), which is
    faster there."""
    monkeypatch.setenv("GRINQH_PREFILL", "tall")


@pytest.fixture(scope="module")
def lib():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from grinqh import _lib
    return _lib.load_library()


def _dev(a, dtype="float16"):
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).to(TORCH_DTYPES[dtype]).cuda()


def _weights(rng, K, N, b, dtype="float16", gs=128, scale_sd=0.02):
    from grinqh.utils import prepare_weight
    W = rand_weight(rng, K, N, b)
    s = to_dtype_np(rng.standard_normal((-(-K // gs), N)) * scale_sd, dtype)
    return W, s, prepare_weight(torch.from_numpy(W).cuda(), b)


def _plan(M, K, N, dtype, b, mode, ldx=None, gs=128, noalloc=False):
    from grinqh import _lib
    dt = _lib.DTYPE_F16 if dtype == "float16" else _lib.DTYPE_BF16
    mc = {"union": _lib.MODE_UNION, "dense": _lib.MODE_DENSE}[mode]
    return _lib.product_kernel(M, K, ldx or K, N, dt, b, gs, mc, noalloc)


def _run(xt, P, st, bt, N, b, t, mode, gs=128):
    from grinqh.kernel import run_product
    return run_product(xt, P, st, bt, b, gs, N // 4, t, mode)


def _noalloc(lib, xt, P, st, bt, N, b, t, mode, gs=128):
    from grinqh import _lib
    M, K = xt.shape
    y = torch.empty((M, N), dtype=xt.dtype, device="cuda")
    dt = _lib.DTYPE_F16 if xt.dtype == torch.float16 else _lib.DTYPE_BF16
    rc = lib.grinqh_gemm_or_gemv_noalloc(
        xt.data_ptr(), M, K, xt.stride(0), N, dt, P.data_ptr(), st.data_ptr(),
        bt.data_ptr() if bt is not None else None, y.data_ptr(), b, gs, _lib.thresholds_f32(t),
        {"union": _lib.MODE_UNION, "dense": _lib.MODE_DENSE}[mode],
        ctypes.c_void_p(torch.cuda.current_stream().cuda_stream))
    _lib.check(rc, "grinqh_gemm_or_gemv_noalloc")
    return y


def _expect(x, W, s, t, b, mode, dtype, bias, gs=128):
    if mode == "dense":
        pre = O.dense_prefill_f64(x, W, s, gs, dtype)
    else:
        pre = O.gemv_union_rounded_f64(x, W, s, t, b, gs, dtype)
    return pre, O.bias_add(pre, bias, dtype)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("max_bits", BITS)
def test_tall_dense(lib, max_bits, dtype):
    """Dense (S9) at 520 rows (two row blocks, the second 8 rows deep: three
    of its four waves hold no row), K = 512 (eight stages, scale groups of
    two), N = 2048, with bias."""
    from grinqh import _lib
    rng = np.random.default_rng(6100 + max_bits)
    M, K, N = 520, 512, 2048
    assert _plan(M, K, N, dtype, max_bits, "dense")[0] == _lib.KERNEL_TALL
    W, s, P = _weights(rng, K, N, max_bits, dtype)
    x = to_dtype_np(rng.standard_normal((M, K)), dtype)
    bias = to_dtype_np(rng.standard_normal(N), dtype)
    y = _run(_dev(x, dtype), P, _dev(s, dtype), _dev(bias, dtype), N, max_bits, [0.0] * 4, "dense")
    pre, fin = _expect(x, W, s, None, max_bits, "dense", dtype, bias)
    assert_output_close(y, pre, fin, dtype, bias=bias, what=f"tall prefill dense b={max_bits} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("max_bits", [4, 8])
@pytest.mark.parametrize("t", [[0.5, 0.1, 2.0, 1.0], [float("inf")] * 4, [-1.0] * 4, [0.0, 0.2, 0.2, 3.0], None],
                         ids=["non_monotone", "skip_all", "all_planes", "tied", "quantiles"])
def test_tall_graded(lib, t, max_bits, dtype):
    """Union grading at 512 rows, K = 1024, N = 1024, with bias: each row of
    K takes the zone set of sigma_k = max_m |x[m][k]| over the whole batch,
    inactive planes masked, the midpoint bias added, RNE(w_eff * s).  Zone
    sets that are not prefixes, none, all, tied thresholds and the 70/20/8/2 %
    quantile mix."""
    rng = np.random.default_rng(6200 + max_bits)
    M, K, N = 512, 1024, 1024
    W, s, P = _weights(rng, K, N, max_bits, dtype)
    x = to_dtype_np(rng.standard_normal((M, K)), dtype)
    if t is None:
        t = [0.0] + np.quantile(O.union_sigma(x), [0.7, 0.9, 0.98]).tolist()
    bias = to_dtype_np(rng.standard_normal(N), dtype)
    y = _run(_dev(x, dtype), P, _dev(s, dtype), _dev(bias, dtype), N, max_bits, t, "union")
    pre, fin = _expect(x, W, s, t, max_bits, "union", dtype, bias)
    assert_output_close(y, pre, fin, dtype, bias=bias, what=f"tall prefill graded t={t} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mode", ["dense", "union"])
def test_tall_split_k_deterministic(lib, mode, dtype):
    """A grid too small for the GPU (512 rows, N = 256: two tiles) splits K
    (4096 rows) into ranges completed in the kernel; the result is held to
    the oracle, equal bit for bit over three calls (the range that finishes
    last changes from call to call, the order of the sum does not), and the
    allocation-free entry point gives the same bits."""
    rng = np.random.default_rng(6300)
    M, K, N, b = 512, 4096, 256, 8
    kern, wm, splits = _plan(M, K, N, dtype, b, mode)
    assert splits > 1, (kern, wm, splits)
    W, s, P = _weights(rng, K, N, b, dtype)
    x = to_dtype_np(rng.standard_normal((M, K)), dtype)
    t = [0.0] + np.quantile(O.union_sigma(x), [0.5, 0.8, 0.95]).tolist()
    bias = to_dtype_np(rng.standard_normal(N), dtype)
    xt, st, bt = _dev(x, dtype), _dev(s, dtype), _dev(bias, dtype)
    ys = [_run(xt, P, st, bt, N, b, t, mode) for _ in range(3)]
    pre, fin = _expect(x, W, s, t, b, mode, dtype, bias)
    assert_output_close(ys[0], pre, fin, dtype, bias=bias, what=f"tall prefill split K {mode} {dtype}")
    for y in ys[1:]:
        assert torch.equal(y, ys[0])
    assert _plan(M, K, N, dtype, b, mode, noalloc=True)[2] == splits
    assert torch.equal(_noalloc(lib, xt, P, st, bt, N, b, t, mode), ys[0])


@pytest.mark.parametrize("dtype", DTYPES)
def test_tall_two_waves_per_block(lib, dtype):
    """256 rows of a wide product (K = 4096, N = 28672) take 256-row blocks
    with K in two ranges; held to the oracle on a
    slice of the columns (the first 1536 and the last 512; columns are
    independent), graded."""
    rng = np.random.default_rng(6400)
    M, K, N, b = 256, 4096, 28672, 8
    kern, wm, splits = _plan(M, K, N, dtype, b, "union")
    assert wm == 256, (kern, wm, splits)
    W, s, P = _weights(rng, K, N, b, dtype)
    x = to_dtype_np(rng.standard_normal((M, K)), dtype)
    t = [0.0] + np.quantile(O.union_sigma(x), [0.7, 0.9, 0.98]).tolist()
    y = _run(_dev(x, dtype), P, _dev(s, dtype), None, N, b, t, "union")
    cols = np.r_[0:1536, N - 512:N]
    pre, fin = _expect(x, W[:, cols], s[:, cols], t, b, "union", dtype, None)
    assert_output_close(y[:, torch.from_numpy(cols).cuda()], pre, fin, dtype, what=f"tall prefill 256-row blocks {dtype}")


@pytest.mark.parametrize("mode,M", [("dense", 512), ("union", 512), ("dense", 2048), ("union", 2048)])
def test_tall_graph_replay_matches_eager(lib, mode, M):
    """The large-batch path (x repack, graded: the grade-word pass, the kernel;
    at 2048 rows the split tiles with their partial sums and counters)
    captured in a HIP graph and replayed several times, with eager calls in
    between, gives the eager result bit for bit on every replay: it enqueues
    only kernels, and every launch leaves the split counters at zero."""
    from grinqh import _lib
    from grinqh.kernel import run_product
    K, N, b = 4096, 28672, 8
    assert _plan(M, K, N, "float16", b, mode)[0] == _lib.KERNEL_TALL
    rng = np.random.default_rng(7100 + M)
    W, s, P = _weights(rng, K, N, b)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    xin, st = _dev(x), _dev(s)
    t = [0.0] + np.quantile(O.union_sigma(x), [0.7, 0.9, 0.98]).tolist() if mode == "union" else [0.0] * 4
    eager = run_product(xin, P, st, None, b, 128, N // 4, t, mode).clone()
    g = torch.cuda.CUDAGraph()
    s_cap = torch.cuda.Stream()
    s_cap.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s_cap):
        run_product(xin, P, st, None, b, 128, N // 4, t, mode)  # sizes this stream's workspace
        torch.cuda.synchronize()
        with torch.cuda.graph(g, stream=s_cap):
            yg = run_product(xin, P, st, None, b, 128, N // 4, t, mode)
    torch.cuda.current_stream().wait_stream(s_cap)
    for i in range(4):
        yg.zero_()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(yg, eager), f"replay {i}: max |diff| {(yg.float() - eager.float()).abs().max().item()}"
        _ = run_product(xin, P, st, None, b, 128, N // 4, t, mode)
        torch.cuda.synchronize()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("mode", ["dense", "union"])
def test_tall_wide_weight_from_129_rows(lib, dtype, mode, monkeypatch):
    """Below 256 rows the default dispatch gives the large-batch kernel the
    weights with at least 192 blocks of 128 columns (Llama-3-8B gate_up, K =
    4096, N = 28672) from 129 rows, and the fused kernel the rest: at 192 rows
    one 256-row block per column block, 64 rows of it past the batch, held to
    the oracle on a slice of the columns (the first 1536 and the last 512;
    columns are independent), with bias; 128 rows stay on the fused kernel."""
    from grinqh import _lib
    monkeypatch.delenv("GRINQH_PREFILL", raising=False)
    rng = np.random.default_rng(6600)
    M, K, N, b = 192, 4096, 28672, 8
    assert _plan(M, K, N, dtype, b, mode)[:2] == (_lib.KERNEL_TALL, 256)
    assert _plan(128, K, N, dtype, b, mode)[0] == _lib.KERNEL_FUSED
    W, s, P = _weights(rng, K, N, b, dtype)
    x = to_dtype_np(rng.standard_normal((M, K)), dtype)
    bias = to_dtype_np(rng.standard_normal(N), dtype)
    t = [0.0] + np.quantile(O.union_sigma(x), [0.7, 0.9, 0.98]).tolist() if mode == "union" else [0.0] * 4
    y = _run(_dev(x, dtype), P, _dev(s, dtype), _dev(bias, dtype), N, b, t, mode)
    cols = np.r_[0:1536, N - 512:N]
    pre, fin = _expect(x, W[:, cols], s[:, cols], t, b, mode, dtype, bias[cols])
    assert_output_close(y[:, torch.from_numpy(cols).cuda()], pre, fin, dtype, bias=bias[cols],
                        what=f"tall prefill 192 rows {mode} {dtype}")


@pytest.mark.parametrize("dtype", DTYPES)
def test_tall_ragged_rows_strided(lib, dtype):
    from grinqh import _lib
    """700 rows (the second 512-row block holds 188: one wave partly, three
    not at all) read from a wider tensor (ldx = K + 64), dense and graded,
    twice in a row."""
    rng = np.random.default_rng(6500)
    M, K, N, b = 700, 384, 1024, 8
    W, s, P = _weights(rng, K, N, b, dtype)
    x = to_dtype_np(rng.standard_normal((M, K)), dtype)
    wide = np.concatenate([x, to_dtype_np(rng.standard_normal((M, 64)), dtype)], axis=1)
    xt = _dev(wide, dtype)[:, :K]
    assert xt.stride(0) == K + 64
    t = [0.0] + np.quantile(O.union_sigma(x), [0.7, 0.9, 0.98]).tolist()
    for mode in ("dense", "union"):
        assert _plan(M, K, N, dtype, b, mode, ldx=K + 64)[0] == _lib.KERNEL_TALL
        pre, fin = _expect(x, W, s, t, b, mode, dtype, None)
        for _ in range(2):
            y = _run(xt, P, _dev(s, dtype), None, N, b, t, mode)
            assert_output_close(y, pre, fin, dtype, what=f"tall prefill ragged strided {mode} {dtype}")


@pytest.mark.parametrize("group_size", [64, 256, 32])
def test_tall_group_sizes(lib, group_size):
    """Scale groups of 64 rows (a new group every stage) and 256 rows (one
    group over four stages) run the large-batch kernel; groups of 32 rows
    (two per stage) take the fused kernel.  Dense, bias, K = 1024."""
    from grinqh import _lib
    rng = np.random.default_rng(6600 + group_size)
    M, K, N, b = 512, 1024, 2048, 8
    kern = _plan(M, K, N, "float16", b, "dense", gs=group_size)[0]
    assert kern == (_lib.KERNEL_FUSED if group_size == 32 else _lib.KERNEL_TALL), kern
    W, s, P = _weights(rng, K, N, b, gs=group_size)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    bias = to_dtype_np(rng.standard_normal(N), "float16")
    y = _run(_dev(x), P, _dev(s), _dev(bias), N, b, [0.0] * 4, "dense", gs=group_size)
    pre, fin = _expect(x, W, s, None, b, "dense", "float16", bias, gs=group_size)
    assert_output_close(y, pre, fin, "float16", bias=bias, what=f"tall prefill group size {group_size}")


def _round_significand(v, bits=11):
    """RNE to `bits` significant bits with no exponent limit (fp16 precision
    without fp16's range)."""
    m, e = np.frexp(np.asarray(v, dtype=np.float64))
    return np.ldexp(np.round(m * 2.0 ** bits) / 2.0 ** bits, e)


def test_tall_scales_beyond_the_fp16_weight_range(lib):
    """fp16 scales of 600-1500 (|w_eff * s| up to ~1.9e5, past 65504), graded:
    a block whose scales reach past 65504 / 2^(max_bits-1) builds the weight
    from s * 2^-e and scales its sums by 2^e, so the result is x @ R(w_eff * s)
    with R fp16's 11-bit rounding without its range limit, finite."""
    from grinqh.utils import prepare_weight
    rng = np.random.default_rng(6700)
    M, K, N, b = 520, 512, 2048, 8
    W = rand_weight(rng, K, N, b)
    P = prepare_weight(torch.from_numpy(W).cuda(), b)
    x = to_dtype_np(rng.standard_normal((M, K)) * 1e-4, "float16")
    s = to_dtype_np(np.where(rng.random((K // 128, N)) < 0.5, -1.0, 1.0) * rng.uniform(600, 1500, (K // 128, N)),
                    "float16")
    bias = to_dtype_np(rng.standard_normal(N), "float16")
    sigma = O.union_sigma(x)
    t = [0.0] + np.quantile(sigma, [0.5, 0.8, 0.95]).tolist()
    y = _run(_dev(x), P, _dev(s), _dev(bias), N, b, t, "union")
    weff = O.effective_weight(W, O.grade(sigma, t, b), b).astype(np.float64)
    pre = x.astype(np.float64) @ _round_significand(weff * np.repeat(s.astype(np.float64), 128, axis=0))
    fin = O.bias_add(pre, bias, "float16")
    assert np.isfinite(fin).all()
    assert_output_close(y, pre, fin, "float16", bias=bias, what="tall prefill, scales past the fp16 weight range")


@pytest.mark.parametrize("splits_wanted", [False, True])
def test_tall_nonfinite_rows(lib, splits_wanted):
    """A NaN or inf activation makes its whole output row NaN (graded), as the
    reference's sum of beta * x does (grinqh/kernel.py:113-114); the other
    rows stay finite -- with K in one range and split."""
    rng = np.random.default_rng(6800)
    M, K, N, b = 520, (4096 if splits_wanted else 256), (256 if splits_wanted else 2048), 8
    assert (_plan(M, K, N, "float16", b, "union")[2] > 1) == splits_wanted
    W, s, P = _weights(rng, K, N, b)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16").copy()
    x[0, 17] = np.nan
    x[M - 1, 200] = np.inf
    y = _run(_dev(x), P, _dev(s), None, N, b, [0.1, 0.5, 1.0, 2.0], "union").float().cpu()
    assert torch.isnan(y[0]).all() and torch.isnan(y[M - 1]).all()
    assert torch.isfinite(y[1:M - 1]).all()


@pytest.mark.parametrize("mode", ["dense", "union"])
def test_tall_gate_up_2048(lib, mode):
    """Llama-3-8B gate_up (K = 4096, N = 28672) at 2048 rows, the configs[2]
    point the bench times: 512-row blocks, 896 tiles of 512 x 128 in row
    block order (224 column blocks each), the first 768 (three full rounds)
    with K in one range, the last 128 (row block 3, word columns 768..1791)
    in two; the first and last 64 rows held to the oracle on a slice of the
    columns that holds both kinds, the graded zone sets from the whole
    batch's statistic.  The allocation-free entry point has no room for the
    partial sums and runs every tile whole: held to the oracle too, and equal
    bit for bit where the workspace call ran whole tiles."""
    from grinqh import _lib
    rng = np.random.default_rng(6900)
    M, K, N, b = 2048, 4096, 28672, 8
    assert _plan(M, K, N, "float16", b, mode)[:3] == (_lib.KERNEL_TALL, 512, 2)
    assert _plan(M, K, N, "float16", b, mode, noalloc=True)[:3] == (_lib.KERNEL_TALL, 512, 1)
    W, s, P = _weights(rng, K, N, b)
    x = to_dtype_np(rng.standard_normal((M, K)), "float16")
    sigma = O.union_sigma(x)
    t = [0.0] + np.quantile(sigma, [0.7, 0.9, 0.98]).tolist() if mode == "union" else [0.0] * 4
    xt, st = _dev(x), _dev(s)
    y = _run(xt, P, st, None, N, b, t, mode)
    rows, cols = np.r_[0:64, M - 64:M], np.r_[0:1024, N - 1024:N]
    ys = y[torch.from_numpy(rows).cuda()][:, torch.from_numpy(cols).cuda()]
    if mode == "dense":
        pre = O.dense_prefill_f64(x[rows], W[:, cols], s[:, cols], 128, "float16")
    else:
        wd = O.graded_weight_rounded(W[:, cols], O.grade(sigma, t, b), s[:, cols], b, 128, "float16")
        pre = x[rows].astype(np.float64) @ wd
    fin = O.bias_add(pre, None, "float16")
    assert_output_close(ys, pre, fin, "float16", what=f"tall prefill gate_up 2048 {mode}")
    record_errors("tall prefill: Llama-3-8B gate_up", f"M={M} {mode}", rows_checked=len(rows),
                  weight_rounded=True, vs_reference=error_stats(ys, fin), vs_own=error_stats(ys, fin))
    yn = _noalloc(lib, xt, P, st, None, N, b, t, mode)
    assert_output_close(yn[torch.from_numpy(rows).cuda()][:, torch.from_numpy(cols).cuda()], pre, fin, "float16",
                        what=f"tall prefill gate_up 2048 {mode} without workspace")
    assert torch.equal(yn[:1536], y[:1536])  # row blocks 0-2: whole tiles
    whole = torch.from_numpy(np.flatnonzero(np.arange(N) % (N // 16) < 768)).cuda()
    assert torch.equal(yn[1536:, whole], y[1536:, whole])  # row block 3, column blocks 0-95
