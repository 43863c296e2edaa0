"""GPU tests of producer fusion (csrc/producer.hip, grinqh/producer.py): the
fused RMSNorm (with and without the residual add) and SiLU*mul against torch
restatements of vLLM's arithmetic, their per-chunk column maxima against the
maxima of their own outputs, and the union product graded from those maxima
against the product that computes the statistic itself (bitwise)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

DT = {"float16": torch.float16, "bfloat16": torch.bfloat16}
U = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}


@pytest.fixture(scope="module", autouse=True)
def _gpu():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")


def _chunk_max(y):
    """Column maxima of |y| per 16-row chunk (NaN ignored unless all NaN)."""
    a = y.float().abs().cpu().numpy()
    M = a.shape[0]
    out = [np.fmax.reduce(a[c:c + 16], axis=0) for c in range(0, M, 16)]
    return np.stack(out)


def _rand(rng, shape, dtype, scale=1.0):
    return torch.from_numpy(rng.standard_normal(shape).astype(np.float32) * scale).to(DT[dtype]).cuda()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("M,K", [(1, 4096), (20, 4096), (64, 1000), (37, 14336)])
@pytest.mark.parametrize("residual", [False, True])
def test_rmsnorm_sigma(M, K, residual, dtype):
    from grinqh.producer import rmsnorm_sigma
    rng = np.random.default_rng(M + K)
    x = _rand(rng, (M, K), dtype, 3.0)
    w = _rand(rng, (K,), dtype)
    r = _rand(rng, (M, K), dtype) if residual else None
    y, sig, h = rmsnorm_sigma(x, w, 1e-5, r)
    torch.cuda.synchronize()
    href = (x.float() + r.float()).to(DT[dtype]) if residual else x
    if residual:
        assert torch.equal(h, href), "residual sum"
    hf = href.float()
    yref = (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5)).to(DT[dtype]).float() * w.float()
    yref = yref.to(DT[dtype]).float()
    # the variance's summation order differs from torch's: one unit of roundoff in two places
    err = (y.float() - yref).abs()
    assert bool((err <= 4 * U[dtype] * yref.abs() + 1e-6).all()), float(err.max())
    np.testing.assert_array_equal(sig.cpu().numpy(), _chunk_max(y))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("M,F", [(1, 14336), (16, 512), (33, 14336), (64, 1032)])
def test_silu_mul_sigma(M, F, dtype):
    from grinqh.producer import silu_mul_sigma
    rng = np.random.default_rng(M * F)
    gu = _rand(rng, (M, 2 * F), dtype, 2.0)
    y, sig = silu_mul_sigma(gu)
    torch.cuda.synchronize()
    g, u = gu[:, :F].float(), gu[:, F:].float()
    act = (g / (1 + torch.exp(-g))).to(DT[dtype]).float()
    yref = (act * u).to(DT[dtype]).float()
    err = (y.float() - yref).abs()
    # exp may differ from torch's by an ulp of fp32: at most one unit of roundoff of act, then of y
    assert bool((err <= 4 * U[dtype] * yref.abs() + 1e-6).all()), float(err.max())
    np.testing.assert_array_equal(sig.cpu().numpy(), _chunk_max(y))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("M", [1, 4, 5, 16, 20, 33, 64, 100])
def test_product_graded_from_producer_statistic(M, dtype):
    """gemv_batch_union_sigma(y, .., sigma_chunks) == grinqh_gemv_batch_union(y, ..)
    bit for bit, including a row with a NaN and one with an inf (the chunk
    maxima ignore NaN the way the products' own statistic does)."""
    from grinqh.kernel import grinqh_gemv_batch_union
    from grinqh.producer import gemv_batch_union_sigma, rmsnorm_sigma
    from grinqh.utils import prepare_weight
    rng = np.random.default_rng(500 + M)
    K, N = 2048, 1536
    x = _rand(rng, (M, K), dtype, 2.0)
    y, sig, _ = rmsnorm_sigma(x, _rand(rng, (K,), dtype))
    if M >= 4:
        y[1, 7] = float("nan")
        y[2, 100] = float("inf")
        from grinqh.producer import _chunks  # recompute the maxima of the edited rows as the producer would
        sig = torch.from_numpy(_chunk_max(y)).cuda()
        assert sig.shape[0] == _chunks(M)
    W = torch.randint(-128, 128, (K, N), dtype=torch.int32).to(torch.int8).cuda()
    P = prepare_weight(W, 8)
    s = (torch.randn(K // 128, N) * 0.01).to(DT[dtype]).cuda()
    sg = y.float().abs().amax(0).cpu().numpy()
    sg = sg[np.isfinite(sg)]
    t = [0.0] + np.quantile(sg, [0.5, 0.8, 0.95]).tolist()
    a = gemv_batch_union_sigma(y, P, s, None, 8, 128, N // 4, t, sig)
    b = grinqh_gemv_batch_union(y, P, s, None, 8, 128, N // 4, t)
    torch.cuda.synchronize()
    assert torch.equal(torch.isnan(a), torch.isnan(b))
    assert torch.equal(torch.nan_to_num(a), torch.nan_to_num(b))
