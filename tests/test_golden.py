"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle still reproduces every stored vector (plane packing, zone bits
and midpoint bias bit-exactly; products through their float64 value).
GPU: the HIP path reproduces them -- packing and grading bit-exactly, graded
GEMV / union batches and the dense product within the stated tolerance.
"""
import glob
import os

import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import TORCH_DTYPES, assert_output_close, dense_rounding_bound

HERE = os.path.dirname(os.path.abspath(__file__))
FILES = sorted(glob.glob(os.path.join(HERE, "golden", "grinqh_*.npz")))
GS = 128


def _meta(path):
    name = os.path.basename(path)[len("grinqh_"):-len(".npz")]
    dtype, b = name.rsplit("_b", 1)
    return dtype, int(b)


def _cases(z):
    return sorted({k[: -len("_thresholds")] for k in z.files if k.endswith("_thresholds")})


def test_fixtures_present():
    assert len(FILES) == 8


@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f) for f in FILES])
def test_oracle_reproduces_fixtures(path):
    dtype, b = _meta(path)
    z = np.load(path)
    W, s = z["W"], z["scale"]
    assert np.array_equal(O.prepare_weight(W, b), z["planes"])
    for key in _cases(z):
        M = int(key.split("_")[0][1:])
        x = z[f"x_m{M}"]
        t = z[f"{key}_thresholds"].tolist()
        bits = O.grade(np.abs(x).max(0).astype(np.float32), t, b)
        assert np.array_equal(bits.astype(np.uint8), z[f"{key}_zone_bits"]), key
        assert np.array_equal(O.midpoint_bias(bits, b).astype(np.int32), z[f"{key}_beta"]), key
        np.testing.assert_allclose(O.gemv_union_f64(x, W, s, t, b, GS), z[f"{key}_y_pre"], rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(O.dense_prefill_f64(z["dense_x"], W, s, GS, dtype), z["dense_y_pre"],
                               rtol=1e-12, atol=1e-12)


def _t(a, dtype):
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(TORCH_DTYPES[dtype]).cuda()


@pytest.mark.gpu
@pytest.mark.parametrize("path", FILES, ids=[os.path.basename(f) for f in FILES])
def test_hip_path_reproduces_fixtures(path):
    from grinqh.kernel import grinqh_gemv_batch_union, run_product
    from grinqh.utils import grade, prepare_weight
    dtype, b = _meta(path)
    z = np.load(path)
    W, s = z["W"], z["scale"]
    N = W.shape[1]
    P = prepare_weight(torch.from_numpy(W).cuda(), b)
    assert np.array_equal(P.cpu().numpy(), z["planes"]), "plane packing"
    st = _t(s, dtype)
    for key in _cases(z):
        M = int(key.split("_")[0][1:])
        xt = _t(z[f"x_m{M}"], dtype)
        t = z[f"{key}_thresholds"].tolist()
        bits, beta = grade(xt, t, b)
        assert np.array_equal(bits.cpu().numpy(), z[f"{key}_zone_bits"]), f"zone bits {key}"
        assert np.array_equal(beta.cpu().numpy(), z[f"{key}_beta"]), f"beta {key}"
        y = grinqh_gemv_batch_union(xt, P, st, None, b, GS, N // 4, t)
        assert_output_close(y, z[f"{key}_y_pre"], z[f"{key}_y"], dtype, what=f"{os.path.basename(path)} {key}")
    x = z["dense_x"]
    y = run_product(_t(x, dtype), P, st, _t(z["dense_bias"], dtype), b, GS, N // 4, [0.0] * 4, "dense")
    assert_output_close(y, z["dense_y_pre"], z["dense_y"], dtype, bias=z["dense_bias"], what="dense",
                        extra_tol=dense_rounding_bound(x, W, s, dtype))
