"""Pins for the CPU oracle (oracle/grinqh_oracle.py).

Each check compares the oracle with something other than its own formula: the
reference tests' identities (tests/test_grinqh_ops.py in the reference), an
independent index derivation (the Marlin converter's address math,
grinqh/kernel.py:393-398), closed forms, torch's own casts, and brute force.
"""
import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O

BITS = [2, 4, 6, 8]


def _rand_w(rng, K, N, b):
    lim = (1 << (b - 1)) - 1
    return rng.integers(-lim - 1, lim + 1, size=(K, N), dtype=np.int64).astype(np.int8)


# --------------------------------------------------------------------------- layout

def test_preshuffle_index_formula_and_inverse():
    rng = np.random.default_rng(1)
    K, N = 5, 320
    W = rng.integers(-128, 128, size=(K, N)).astype(np.int8)
    P = O.preshuffle(W)
    for c in range(N // 16):
        for r in range(16):
            assert np.array_equal(P[:, 16 * c + r], W[:, r * (N // 16) + c])
    assert np.array_equal(O.postshuffle(P), W)
    with pytest.raises(AssertionError):
        O.preshuffle(np.zeros((2, 40), np.int8))


@pytest.mark.parametrize("b", BITS)
def test_pack_unpack_roundtrip_and_size(b):
    """tests/test_grinqh_ops.py:58-88 restated: storage = numel*b/8, per-row and
    vectorised unpack equal, and unpack(pack(A)) == A >> (8-b)."""
    rng = np.random.default_rng(b)
    K, N = 384, 320
    A = rng.integers(0, 256, size=(K, N), dtype=np.int64).astype(np.uint8)
    B = O.pack_planes(A, b)
    assert B.nbytes == A.size * b // 8
    rec = np.stack([O.unpack_planes(B, i, b // 2, N // 4).view(np.uint8)[0] for i in range(K)])
    vec = O.unpack_planes(B, np.arange(K), b // 2, N // 4).view(np.uint8)
    assert np.array_equal(rec, vec)
    assert np.array_equal(vec, A >> (8 - b))


@pytest.mark.parametrize("b", BITS)
def test_plane_layout_matches_marlin_index_math(b):
    """Independent derivation of S2+S4: the Marlin converter addresses logical
    column n of row k at word (k, n % (N/16) [+ plane offset]) and bit
    (lane%4)*8 + (3 - lane//4)*2 with lane = n // (N/16) (grinqh/kernel.py:393-412).
    Assemble every code from those addresses and compare with W."""
    rng = np.random.default_rng(10 + b)
    K, N = 64, 256
    W = _rand_w(rng, K, N, b)
    B = O.prepare_weight(W, b)
    Z = b // 2
    ng = N // 16
    n = np.arange(N)
    grp = n % ng
    lane = n // ng
    shift = ((lane % 4) * 8 + (3 - lane // 4) * 2).astype(np.uint32)
    code = np.zeros((K, N), np.int64)
    for z in range(Z):
        plane = B[:, z * ng + grp]
        code = (code << 2) | ((plane >> shift[None, :]) & 3)
    expect = W.astype(np.int64) & ((1 << b) - 1)
    assert np.array_equal(code, expect)


@pytest.mark.parametrize("b", BITS)
def test_decode_weight_inverts_prepare(b):
    rng = np.random.default_rng(20 + b)
    W = _rand_w(rng, 96, 160, b)
    assert np.array_equal(O.decode_weight(O.prepare_weight(W, b), b, 160 // 4), W)


# --------------------------------------------------------------------------- grading

def test_grade_uses_fp32_threshold_and_strict_gt():
    # t just below 1.0 in double rounds to 1.0 in fp32 -> |x| == 1.0 is NOT above it
    t = [1.0 - 1e-12, 0.5, 2.0, -1.0]
    bits = O.grade(np.array([1.0, -1.0, 0.75, np.nan, np.inf, -0.0], np.float16), t, 8)
    assert [int(v) for v in bits] == [
        0b1010, 0b1010, 0b1010, 0, 0b1111, 0b1000]
    # numpy fp64 comparison would differ on the first element
    assert 1.0 > t[0]


def test_grade_bruteforce_all_fp16():
    vals = np.arange(0, 1 << 16, dtype=np.uint32).astype(np.uint16).view(np.float16)
    t = [0.3, 1.7, 65504.0, 0.0]
    bits = O.grade(vals, t, 8)
    a = np.abs(vals.astype(np.float64))
    for z, tz in enumerate(t):
        tz32 = float(np.float32(tz))
        with np.errstate(invalid="ignore"):
            ok = a > tz32
        assert np.array_equal(((bits >> z) & 1).astype(bool), ok)


@pytest.mark.parametrize("b", BITS)
def test_grade_special_cases(b):
    rng = np.random.default_rng(3)
    x = rng.standard_normal(256).astype(np.float16)
    assert np.all(O.grade(x, [-1.0] * 4, b) == (1 << (b // 2)) - 1)
    q1 = float(np.quantile(np.abs(x).astype(np.float32), 1.0))
    assert np.all(O.grade(x, [q1] * 4, b) == 0)


def test_union_sigma_nan_and_padding_rule():
    """union_sigma against its two sources.  (1) Triton's tl.max: its combine
    is tl.maximum at the default propagate_nan, which lowers to maxnum (NaN
    ignored); read from the installed Triton (the reference pins 3.7.1 in
    uv.lock, absent here).  (2) The batch tile of next_power_of_2(M) rows with
    zero padding: brute force over tiny batches by an explicit tile."""
    triton = pytest.importorskip("triton")
    import inspect
    from triton.language import core, standard
    from triton.language.semantic import TritonSemantic
    assert "core.maximum(a, b)" in inspect.getsource(standard._elementwise_max.fn)
    assert inspect.signature(core.maximum).parameters["propagate_nan"].default == core.PropagateNan.NONE
    src = inspect.getsource(TritonSemantic.maximum)
    assert src.index("PropagateNan.NONE") < src.index("create_maxnumf") < src.index("raise ValueError")
    assert triton.__version__.startswith("3.")

    def maxnum(a, b):  # IEEE maxNum: a NaN operand loses to a number
        return b if np.isnan(a) else a if np.isnan(b) else max(a, b)

    rng = np.random.default_rng(3)
    for M in range(1, 10):
        for _ in range(20):
            x = rng.standard_normal((M, 5))
            x[rng.random((M, 5)) < 0.4] = np.nan
            x[:, 0] = np.nan  # one column all NaN
            B = 1 << (M - 1).bit_length()
            tile = np.zeros((B, 5))
            tile[:M] = x
            exp = np.empty(5)
            for k in range(5):
                acc = abs(tile[0, k])
                for m in range(1, B):
                    acc = maxnum(acc, abs(tile[m, k]))
                exp[k] = acc
            np.testing.assert_array_equal(O.union_sigma(x), exp)
        assert np.isnan(O.union_sigma(np.full((M, 1), np.nan))[0]) == (M & (M - 1) == 0)


@pytest.mark.parametrize("b", BITS)
def test_effective_weight_prefix_closed_form(b):
    """Prefix of `a` active zones keeps the top 2a bits and adds the midpoint of
    the dropped bits: floor(c / 2^(b-2a)) * 2^(b-2a) + 2^(b-2a-1)."""
    Z = b // 2
    c = np.arange(-(1 << (b - 1)), 1 << (b - 1), dtype=np.int64)
    W = c.astype(np.int8).reshape(-1, 1)
    for a in range(Z + 1):
        bits = np.full(W.shape[0], (1 << a) - 1, np.uint8)
        got = O.effective_weight(W, bits, b)[:, 0]
        if a == 0:
            want = np.zeros_like(c)
        elif a == Z:
            want = c
        else:
            q = 1 << (b - 2 * a)
            want = np.floor_divide(c, q) * q + q // 2
        assert np.array_equal(got, want), a


def test_effective_weight_nonprefix_mask_matches_reference_test_oracle():
    """Non-monotone thresholds give non-prefix masks; restate the reference test
    oracle literally (tests/test_grinqh_ops.py:36-55) with torch and compare."""
    rng = np.random.default_rng(7)
    for b in BITS:
        W = _rand_w(rng, 64, 32, b)
        x = rng.standard_normal((1, 64)).astype(np.float16)
        t = [0.9, 0.1, 1.5, 0.0]
        got = O.masked_weight_ref(W, x, t, b)

        wt = torch.from_numpy(W)
        xt = torch.from_numpy(x)
        shift_amt = 8 - b
        x_abs = xt.abs().float().flatten()
        w_u8 = (wt << shift_amt).view(torch.uint8)
        row_mask = torch.zeros_like(x_abs, dtype=torch.uint8)
        bias = torch.zeros_like(x_abs, dtype=torch.float32)
        prev = 0
        for zone in range(b // 2):
            active = x_abs > t[zone]
            row_mask |= active.to(torch.uint8) * (0xC0 >> 2 * zone)
            cur = (1 << (b - 1)) >> (2 * zone + 2)
            bias += active * (cur - prev)
            prev = cur
        ref = (w_u8 & row_mask[:, None]).view(torch.int8).float() / 2 ** shift_amt + bias[:, None]
        assert np.array_equal(got, ref.double().numpy())


# --------------------------------------------------------------------------- products

def test_bf16_cast_matches_torch():
    rng = np.random.default_rng(4)
    y = np.concatenate([rng.standard_normal(10000) * 10.0 ** rng.integers(-6, 6, 10000),
                        [0.0, -0.0, np.inf, -np.inf, 3.0e38]])
    ours = O.rne_cast(y, "bfloat16")
    ref = torch.from_numpy(y.astype(np.float32)).to(torch.bfloat16).double().numpy()
    assert np.array_equal(ours, ref)
    ours16 = O.rne_cast(y, "float16")
    ref16 = torch.from_numpy(y.astype(np.float32)).half().double().numpy()
    assert np.array_equal(ours16, ref16)


@pytest.mark.parametrize("b", BITS)
def test_gemv_all_active_is_dense_fp32(b):
    """tests/test_grinqh_ops.py:156-190: thresholds -1 -> the GEMV equals
    X @ (W * s) (fp32 in the reference; float64 here)."""
    rng = np.random.default_rng(5)
    W = _rand_w(rng, 256, 256, b)
    x = rng.standard_normal((1, 256)).astype(np.float16)
    s = rng.standard_normal((2, 256)).astype(np.float16)
    y = O.gemv_f64(x, W, s, [-1.0] * 4, b, 128)
    ref = x.astype(np.float64) @ (W.astype(np.float64) * np.repeat(s.astype(np.float64), 128, 0))
    np.testing.assert_allclose(y, ref, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("b", BITS)
def test_gemv_skip_all_is_zero(b):
    rng = np.random.default_rng(6)
    W = _rand_w(rng, 256, 256, b)
    x = rng.standard_normal((1, 256)).astype(np.float16)
    s = rng.standard_normal((2, 256)).astype(np.float16)
    q = float(np.quantile(np.abs(x).astype(np.float32), 1.0))
    y = O.gemv(x, W, s, None, [q] * 4, b, 128)
    assert np.all(y == 0)


def test_gemv_bruteforce_tiny():
    """Brute-force S8 element by element from the zone rule on a tiny case."""
    rng = np.random.default_rng(8)
    b, K, N = 8, 32, 16
    W = _rand_w(rng, K, N, b)
    x = rng.standard_normal((1, K)).astype(np.float16)
    s = (rng.random((1, N)) + 0.5).astype(np.float16)
    t = [0.2, 0.6, 1.1, 1.9]
    y = O.gemv_f64(x, W, s, t, b, 128)
    for n in range(N):
        acc = 0.0
        for k in range(K):
            xv = float(x[0, k])
            a = sum(1 for z in range(4) if np.float32(abs(xv)) > np.float32(t[z]))
            prefix = all(np.float32(abs(xv)) > np.float32(t[z]) for z in range(a))
            assert prefix  # thresholds are increasing here
            c = int(W[k, n])
            if a == 0:
                w = 0
            elif a == 4:
                w = c
            else:
                q = 1 << (8 - 2 * a)
                w = (c // q) * q + q // 2
            acc += xv * w * float(s[0, n])
        assert abs(acc - y[0, n]) <= 1e-9 * max(1.0, abs(acc))


@pytest.mark.parametrize("b", BITS)
@pytest.mark.parametrize("B", [2, 3, 5, 8])
def test_union_identities(b, B):
    """tests/test_grinqh_ops.py:245-282: at all-active thresholds the union GEMV
    equals the looped per-row GEMV and the dense masked reference."""
    rng = np.random.default_rng(9)
    W = _rand_w(rng, 256, 256, b)
    x = rng.standard_normal((B, 256)).astype(np.float16)
    s = rng.standard_normal((2, 256)).astype(np.float16)
    t = [-1.0] * 4
    yu = O.gemv_union_f64(x, W, s, t, b, 128)
    yl = np.concatenate([O.gemv_f64(x[i:i + 1], W, s, t, b, 128) for i in range(B)])
    np.testing.assert_allclose(yu, yl, rtol=1e-12, atol=1e-9)
    # the union statistic is the column max of |x|
    tq = [0.5, 1.0, 1.5, 2.0]
    bits_u = O.grade(np.abs(x.astype(np.float32)).max(0), tq, b)
    wm = O.effective_weight(W, bits_u, b).astype(np.float64)
    ref = x.astype(np.float64) @ (wm * np.repeat(s.astype(np.float64), 128, 0))
    np.testing.assert_allclose(O.gemv_union_f64(x, W, s, tq, b, 128), ref, rtol=1e-12, atol=1e-9)


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("b", BITS)
def test_dense_weight_elementwise_rne(dtype, b):
    """S9 elementwise W*s rounded in the activation dtype, checked against
    torch's own CPU multiply in that dtype (tests/test_grinqh_ops.py:106)."""
    rng = np.random.default_rng(11)
    W = _rand_w(rng, 256, 64, b)
    s = rng.standard_normal((2, 64)).astype(np.float32)
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    st = torch.from_numpy(s).to(tdt)
    ref = (torch.from_numpy(W).to(tdt) * st.repeat_interleave(128, 0)).double().numpy()
    got = O.dense_weight(W, st.double().numpy(), 128, dtype)
    assert np.array_equal(got, ref)


def test_dispatch_shapes():
    rng = np.random.default_rng(12)
    W = _rand_w(rng, 128, 64, 8)
    s = rng.standard_normal((1, 64)).astype(np.float16)
    x = rng.standard_normal((2, 3, 128)).astype(np.float16)
    y = O.gemm_or_gemv(x, W, s, None, 8, 128, [0.1] * 4)
    assert y.shape == (2, 3, 64)
    np.testing.assert_array_equal(y.reshape(6, 64), O.dense_prefill(x.reshape(6, 128), W, s, None, 128))
    y1 = O.gemm_or_gemv(x[:1, :1], W, s, None, 8, 128, [0.1] * 4)
    np.testing.assert_array_equal(y1.reshape(1, 64), O.gemv(x[0, :1], W, s, None, [0.1] * 4, 8, 128))


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
@pytest.mark.parametrize("b", BITS)
def test_graded_weight_rounded_against_torch(dtype, b):
    """RNE(w_eff * s): the effective integer weight (already pinned above) times
    the scale in fp32 -- exact, since |w_eff| < 2^9 and s has at most 11
    significant bits -- then torch's own cast to the activation dtype.  With
    every zone active it equals S9's dense weight."""
    rng = np.random.default_rng(13 + b)
    K, N = 256, 96
    W = _rand_w(rng, K, N, b)
    tdt = torch.float16 if dtype == "float16" else torch.bfloat16
    s = torch.from_numpy(rng.standard_normal((2, N)).astype(np.float32) * 3).to(tdt)
    x = rng.standard_normal(K).astype(np.float32)
    t = [0.3, 0.9, 1.4, 2.2]
    bits = O.grade(x, t, b)
    weff = torch.from_numpy(O.effective_weight(W, bits, b).astype(np.float32))
    ref = (weff * s.float().repeat_interleave(128, 0)).to(tdt).double().numpy()
    got = O.graded_weight_rounded(W, bits, s.double().numpy(), b, 128, dtype)
    assert np.array_equal(got, ref)
    all_bits = O.grade(x, [-1.0] * 4, b)
    assert np.array_equal(O.graded_weight_rounded(W, all_bits, s.double().numpy(), b, 128, dtype),
                          O.dense_weight(W, s.double().numpy(), 128, dtype))


def test_rounded_union_product_and_dense_exact():
    """The rounded S10 product is x @ RNE(w_eff*s); the exact dense product is
    the all-zones S10 (tests/test_grinqh_ops.py:170, 190); with every zone
    active the rounded S10 is S9 (grinqh/kernel.py:586-587)."""
    rng = np.random.default_rng(14)
    W = _rand_w(rng, 256, 64, 8)
    x = rng.standard_normal((3, 256)).astype(np.float16)
    s = rng.standard_normal((2, 64)).astype(np.float16)
    np.testing.assert_allclose(O.dense_exact_f64(x, W, s, 128), O.gemv_union_f64(x, W, s, [-1.0] * 4, 8, 128),
                               rtol=1e-12, atol=1e-9)
    np.testing.assert_array_equal(O.gemv_union_rounded_f64(x, W, s, [-1.0] * 4, 8, 128, "float16"),
                                  O.dense_prefill_f64(x, W, s, 128, "float16"))
    t = [0.0, 0.5, 1.0, 2.0]
    sigma = np.abs(x.astype(np.float32)).max(0)
    wr = O.graded_weight_rounded(W, O.grade(sigma, t, 8), s, 8, 128, "float16")
    np.testing.assert_array_equal(O.gemv_union_rounded_f64(x, W, s, t, 8, 128, "float16"),
                                  x.astype(np.float64) @ wr)


@pytest.mark.parametrize("b", [4, 8])
def test_cpu_reference_matches_oracle(b):
    """The CPU baseline (oracle/cpu_reference.py, torch eager) computes what
    the oracle does: the same int8 weights from the planes, S10 graded math and
    S9 dense math on the same inputs."""
    from oracle import cpu_reference as C
    rng = np.random.default_rng(15 + b)
    K, N, M = 256, 192, 5
    W = _rand_w(rng, K, N, b)
    P = torch.from_numpy(O.prepare_weight(W, b).view(np.int32))
    x = rng.standard_normal((M, K)).astype(np.float16)
    s = (rng.standard_normal((K // 128, N)) * 0.05).astype(np.float16)
    assert np.array_equal(C.weight_int8(P, b).numpy(), W)
    t = [0.0] + np.quantile(np.abs(x).astype(np.float32).max(0), [0.5, 0.8, 0.95]).tolist()
    yg = C.graded(torch.from_numpy(x), P, torch.from_numpy(s), t, 128, b).double().numpy()
    ref = O.gemv_union(x, W, s, None, t, b, 128, "float16")
    np.testing.assert_allclose(yg, ref, rtol=2e-3, atol=2e-3 * np.sqrt(np.mean(ref ** 2)))
    yd = C.dense_prefill(torch.from_numpy(x), P, torch.from_numpy(s), 128, b).double().numpy()
    refd = O.dense_prefill(x, W, s, None, 128, "float16")
    np.testing.assert_allclose(yd, refd, rtol=2e-3, atol=2e-3 * np.sqrt(np.mean(refd ** 2)))


# --------------------------------------------------------------------------- epilogue

_TDT = {"float16": torch.float16, "bfloat16": torch.bfloat16}
# an exact sum and a bias whose cast-then-add result (two roundings) differs
# from one rounding of their sum: fp16 has 11 significant bits, so 2049 lies
# halfway between 2048 and 2050 and rounds to 2048, and 2048 + 1 rounds to
# 2048 again, where 2049 + 1 = 2050 is exact; bf16 (8 bits) likewise at 257
_TWICE_CASES = {"float16": [(2049.0, 1.0, 2048.0, 2050.0), (-2051.0, -1.0, -2052.0, -2052.0),
                            (4097.0, 3.0, 4100.0, 4100.0), (2051.0, 1.0, 2052.0, 2052.0),
                            (1025.5, 0.5, 1026.0, 1026.0), (2049.0, 2.0, 2050.0, 2052.0)],
                "bfloat16": [(257.0, 1.0, 256.0, 258.0), (-513.0, -2.0, -512.0, -516.0),
                             (259.0, 1.0, 260.0, 260.0), (257.0, 3.0, 260.0, 260.0)]}


def _torch_cast_then_add(y32: np.ndarray, bias: np.ndarray, dtype: str) -> np.ndarray:
    """The reference epilogue in torch on the CPU: the fp32 result cast to the
    activation dtype, then ``add_`` of the bias in that dtype
    (grinqh/kernel.py:706-708)."""
    y = torch.from_numpy(np.asarray(y32, dtype=np.float32)).to(_TDT[dtype])
    if bias is not None:
        y.add_(torch.from_numpy(np.asarray(bias, dtype=np.float32)).to(_TDT[dtype]))
    return y.double().numpy()


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_bias_add_is_cast_then_add(dtype):
    """O.bias_add against torch's cast-then-add on random fp32 results over
    many magnitudes (and zeros, infinities), plus targeted values where the two
    roundings differ from one: the oracle must give the two-rounding value."""
    rng = np.random.default_rng(21)
    n = 20000
    y = (rng.standard_normal(n) * 10.0 ** rng.integers(-4, 5, n)).astype(np.float32)
    y[:4] = [0.0, -0.0, np.inf, -np.inf]
    bias = torch.from_numpy((rng.standard_normal(n) * 10.0 ** rng.integers(-4, 5, n)).astype(np.float32))
    bias = bias.to(_TDT[dtype]).float().numpy()
    got = O.bias_add(y.astype(np.float64)[None, :], bias, dtype)[0]
    ref = _torch_cast_then_add(y, bias, dtype)
    assert np.array_equal(got, ref, equal_nan=True)
    assert np.array_equal(O.bias_add(y.astype(np.float64)[None, :], None, dtype)[0],
                          _torch_cast_then_add(y, None, dtype))
    for v, b, twice, once in _TWICE_CASES[dtype]:
        yy, bb = np.array([[v]]), np.array([b])
        assert O.bias_add(yy, bb, dtype)[0, 0] == twice == _torch_cast_then_add(np.float32([v]), bb, dtype)[0]
        assert O.rne_cast(np.array([v + b]), dtype)[0] == once
    # the targeted cases are discriminating: at least one of them differs
    assert any(tw != on for _, _, tw, on in _TWICE_CASES[dtype])


@pytest.mark.parametrize("dtype", ["float16", "bfloat16"])
def test_gemv_and_dense_prefill_bias_against_torch(dtype):
    """The oracle's products with a bias, compared with torch on the CPU on
    integer operands whose fp32 sums are exact (so no summation order enters):
    O.gemv against the fp32 GEMV result cast then bias-added
    (grinqh/kernel.py:697-708), O.dense_prefill against torch's
    ``x @ Wd`` in the activation dtype followed by ``y.add_(bias)``
    (:561-587, :707-708).  The operands put many results where the two
    roundings differ from one, which the test also counts."""
    rng = np.random.default_rng(22)
    K, N, b = 256, 256, 8
    W = _rand_w(rng, K, N, b)
    s = np.full((K // 128, N), 1.0, dtype=np.float64)
    x = rng.integers(-3, 4, size=(6, K)).astype(np.float64)
    bias = rng.integers(-5, 6, size=N).astype(np.float64)
    tdt = _TDT[dtype]
    # GEMV (one row, thresholds -1: every zone active, w_eff = W)
    exact = x[:1] @ W.astype(np.float64)
    got = O.gemv(x[:1], W, s, bias, [-1.0] * 4, b, 128, dtype)
    assert np.array_equal(got, _torch_cast_then_add(exact.astype(np.float32), bias, dtype))
    # dense prefill: torch CPU matmul in the activation dtype, then add_ in that dtype
    Wd = torch.from_numpy(W.astype(np.float32)).to(tdt)
    y_t = torch.from_numpy(x.astype(np.float32)).to(tdt) @ Wd
    y_t.add_(torch.from_numpy(bias.astype(np.float32)).to(tdt))
    got = O.dense_prefill(x, W, s, bias, 128, dtype)
    assert np.array_equal(got, y_t.double().numpy())
    once = O.rne_cast(x @ W.astype(np.float64) + bias[None, :], dtype)
    assert int((once != got).sum()) > 20
