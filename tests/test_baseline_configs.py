"""GPU parity tests at every BASELINE.json configuration point, with the
benchmark's own synthetic inputs.

In the style of the reference's tests/test_grinqh_ops.py:193-282 (thresholds
from quantiles of the activations, graded product against a masked dense
reference), at the shapes and batch sizes of BASELINE configs[1], [2] and [4]:

* Llama-3-8B qkv / o_proj / gate_up / down x M in {1, 4, 16, 64},
  union grading with t = [0, P50, P80, P95] of sigma_k = max_m |x[m,k]|;
* the same shapes at M in {512, 2048, 8192}, t = [0, P70, P90,
  P98] (70/20/8/2 % of rows at 1/2/3/4 planes), plus the reference's dense
  dispatch at M = 2048;
* Llama-3-70B qkv / gate_up / down at M in {1, 64, 4096} with
  thresholds -1 (every plane of every row).

Inputs follow bench.py: x ~ N(0,1) with 1 % of channels x20 (fp16); weights
0.02*N(0,1) RTN-quantised per 128-row group to int8 codes with fp16 scales
(the 70B shapes use uniform codes and N(0, 0.05) scales, which bounds the
oracle's memory).  Every output row is held to the float64 oracle up to 64
rows; larger batches hold 64 rows (the first 32 and the last 32) to it, with
the statistic and grades computed from the whole batch.  Each kernel is held
to the product it computes with the base tolerance: S10 (scale in fp32) for
the kernels that apply the scale after the sum, S10 with RNE(w_eff*s) for the
kernels that round the scaled weight first (as S9 does, grinqh/kernel.py:586).
Every case is also held to the reference's own semantics (S10 for union
grading, S9 for the dense dispatch): with the base tolerance plus the bound
the rounding of the scaled weight to the activation dtype can make,
u * (|x| @ |w_eff * s|) (one unit of roundoff per weight), since exactly one
of the two products rounds the weight.  Both errors are recorded per case
(GRINQH_PARITY_LOG).
"""
import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import UNIT_ROUNDOFF, assert_output_close, error_stats, record_errors, rounds_weight

pytestmark = pytest.mark.gpu

SHAPES_8B = [("qkv", 4096, 6144), ("o_proj", 4096, 4096), ("gate_up", 4096, 28672), ("down", 14336, 4096)]
SHAPES_70B = [("qkv", 8192, 10240), ("gate_up", 8192, 57344), ("down", 28672, 8192)]
GS, B = 128, 8
ROWS_HELD = 64
COL_CHUNK = 8192


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    from grinqh import _lib
    _lib.load_library()


_weights = {}


def weights(name, K, N, seed, kind="rtn"):
    """(planes on the GPU, scales on the GPU, W int8 [K,N] and scales on the CPU), cached per shape."""
    key = (name, K, N)
    if key not in _weights:
        from grinqh.utils import prepare_weight
        dev = torch.device("cuda:0")
        if kind == "rtn":
            from bench import synth_weight
            w, s = synth_weight(torch, K, N, seed, dev)
        else:
            g = torch.Generator(device=dev).manual_seed(seed)
            w = torch.randint(-128, 128, (K, N), generator=g, device=dev, dtype=torch.int32).to(torch.int8)
            s = (0.05 * torch.randn((K // GS, N), generator=g, device=dev)).half()
        P = prepare_weight(w, B)
        _weights.clear()  # one shape at a time keeps host and device memory small
        _weights[key] = (P, s, w.cpu().numpy(), s.double().cpu().numpy())
        del w
    return _weights[key]


def synth_x(M, K, seed):
    from bench import synth_x as bx
    return bx(torch, M, K, seed, torch.device("cuda:0"))


def held_rows(M):
    if M <= ROWS_HELD:
        return np.arange(M)
    return np.concatenate([np.arange(ROWS_HELD // 2), np.arange(M - ROWS_HELD // 2, M)])


def oracle_rows(x_rows, sigma, W, s, t, dtype, graded, rounded):
    """Float64 products of the held rows, column chunk by column chunk: the
    kernel's own product (``own``), the reference's (``ref``: S10 for
    graded, S9 for dense) and the weight-rounding bound between the two,
    ``u * (|x| @ |w_eff * s|)``."""
    K, N = W.shape
    xr = x_rows.astype(np.float64)
    bits = O.grade(sigma, t, B) if graded else O.grade(sigma, [-1.0] * 4, B)
    own = np.empty((xr.shape[0], N))
    ref = np.empty((xr.shape[0], N))
    bound = np.empty((xr.shape[0], N))
    for c0 in range(0, N, COL_CHUNK):
        c1 = min(N, c0 + COL_CHUNK)
        Wc, sc = W[:, c0:c1], s[:, c0:c1]
        weff = O.effective_weight(Wc, bits, B).astype(np.float64) * np.repeat(sc, GS, 0)[:K]
        bound[:, c0:c1] = UNIT_ROUNDOFF[dtype] * (np.abs(xr) @ np.abs(weff))
        if graded:
            exact = xr @ weff
            ref[:, c0:c1] = exact
            own[:, c0:c1] = xr @ O.graded_weight_rounded(Wc, bits, sc, B, GS, dtype) if rounded else exact
        else:
            r9 = xr @ O.dense_weight(Wc, sc, GS, dtype)
            ref[:, c0:c1] = r9
            own[:, c0:c1] = r9 if rounded else O.dense_exact_f64(xr, Wc, sc, GS)
    return own, ref, bound


def run_case(config, name, K, N, M, x, t, mode, wts):
    from grinqh.kernel import run_product
    P, s_dev, W, s = wts
    y = run_product(x, P, s_dev, None, B, GS, N // 4, t, mode)
    torch.cuda.synchronize()
    rows = held_rows(M)
    xn = x[torch.from_numpy(rows).cuda()].double().cpu().numpy()
    sigma = x.abs().float().amax(0).cpu().numpy()  # exact; these inputs hold no NaN
    graded = mode == "union"
    rounded = rounds_weight(M)
    own, ref, bound = oracle_rows(xn, sigma, W, s, t, "float16", graded, rounded)
    yr = y[torch.from_numpy(rows).cuda()]
    fin_own = O.bias_add(own, None, "float16")
    fin_ref = O.bias_add(ref, None, "float16")
    case = f"{name} K={K} N={N} M={M} {mode}"
    assert_output_close(yr, own, fin_own, "float16", what=case)
    # the reference's product (S10 / S9), with the weight-rounding bound
    assert_output_close(yr, ref, fin_ref, "float16", extra_tol=bound, what=case + " against the reference")
    e_own = error_stats(yr, fin_own)
    e_ref = error_stats(yr, fin_ref)
    record_errors(config, case, rows_checked=int(len(rows)), weight_rounded=bool(rounded),
                  vs_own=e_own, vs_reference=e_ref)
    return e_own


@pytest.mark.parametrize("M", [1, 4, 16, 64])
@pytest.mark.parametrize("shape", SHAPES_8B, ids=[s[0] for s in SHAPES_8B])
def test_config1_decode_sweep(shape, M):
    """union grading at the 50/80/95th percentiles of sigma."""
    name, K, N = shape
    wts = weights(name, K, N, 1000 + SHAPES_8B.index(shape))
    x = synth_x(M, K, 17 * SHAPES_8B.index(shape) + M)
    sigma = x.abs().float().amax(0).cpu().numpy()
    t = [0.0] + np.quantile(sigma, [0.5, 0.8, 0.95]).tolist()
    run_case("configs[1] decode sweep", name, K, N, M, x, t, "union", wts)


@pytest.mark.parametrize("M", [512, 2048, 8192])
@pytest.mark.parametrize("shape", SHAPES_8B, ids=[s[0] for s in SHAPES_8B])
def test_config2_prefill_sweep(shape, M):
    """union grading with the 70/20/8/2 % grade mix."""
    name, K, N = shape
    wts = weights(name, K, N, 1000 + SHAPES_8B.index(shape))
    x = synth_x(M, K, 199 + SHAPES_8B.index(shape))
    sigma = x.abs().float().amax(0).cpu().numpy()
    t = [0.0] + np.quantile(sigma, [0.7, 0.9, 0.98]).tolist()
    bits = O.grade(sigma, t, B)
    mix = np.bincount(np.array([bin(int(v)).count("1") for v in bits]), minlength=5)[1:] / len(bits)
    assert abs(mix[0] - 0.7) < 0.01 and abs(mix[3] - 0.02) < 0.01, mix
    run_case("configs[2] prefill sweep", name, K, N, M, x, t, "union", wts)


@pytest.mark.parametrize("shape", SHAPES_8B, ids=[s[0] for s in SHAPES_8B])
def test_config2_dense_dispatch(shape):
    """The reference's own dispatch for more than one row (dense S9,
    grinqh/kernel.py:663-680) at 2048 rows of the configs[2] shapes."""
    name, K, N = shape
    wts = weights(name, K, N, 1000 + SHAPES_8B.index(shape))
    x = synth_x(2048, K, 99 + SHAPES_8B.index(shape))
    run_case("configs[2] dense dispatch", name, K, N, 2048, x, [0.0] * 4, "dense", wts)


@pytest.mark.parametrize("M", [1, 64, 4096])
@pytest.mark.parametrize("shape", SHAPES_70B, ids=[s[0] for s in SHAPES_70B])
def test_config4_llama70b_adversarial(shape, M):
    """every token above every threshold (t = -1), so
    every plane of every row is read (tests/test_grinqh_ops.py:187)."""
    name, K, N = shape
    wts = weights("70b-" + name, K, N, 2000 + SHAPES_70B.index(shape), kind="uniform")
    x = synth_x(M, K, 299 + SHAPES_70B.index(shape))
    run_case("configs[4] Llama-3-70B adversarial", name, K, N, M, x, [-1.0] * 4, "union", wts)
