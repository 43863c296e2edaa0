"""Shared test helpers: seeded inputs in the reference tests' style and the
output tolerance used by every floating-point parity check."""
from __future__ import annotations

import json
import os

import numpy as np
import torch

# Unit roundoff of the output dtypes.
UNIT_ROUNDOFF = {"float16": 2.0 ** -11, "bfloat16": 2.0 ** -8}
TORCH_DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16}


def rand_weight(rng: np.random.Generator, K: int, N: int, b: int) -> np.ndarray:
    """Uniform b-bit signed codes (reference tests: torch.randint(-limit-1, limit+1))."""
    lim = (1 << (b - 1)) - 1
    return rng.integers(-lim - 1, lim + 1, size=(K, N), dtype=np.int64).astype(np.int8)


def to_dtype_np(a: np.ndarray, dtype: str) -> np.ndarray:
    """Round float64/float32 values into fp16/bf16 and back to float64 (RNE)."""
    return torch.from_numpy(np.asarray(a, dtype=np.float32)).to(TORCH_DTYPES[dtype]).double().numpy()


def rounds_weight(M: int, dtype: str = "float16") -> bool:
    """Whether the kernel serving an M-row batch rounds w_eff*s to the
    activation dtype (as the reference's dense path does, grinqh/kernel.py:586)
    instead of applying the scale in fp32 after the sum: the prefill kernels
    above 64 rows, and the fp16 decode kernel for 17-64 rows."""
    return M > 64 or (M > 16 and dtype == "float16")


def own_product(x, W, s, t, b, gs, dtype, graded):
    """Float64 product the kernel serving this batch computes: S10 (graded) or
    the exact dense product when it applies the scale after the sum, the same
    with RNE(w_eff*s) -- S9 for the dense dispatch -- when it rounds the
    scaled weight first.  Kernels are held to it with the base tolerance."""
    from oracle import grinqh_oracle as O
    M = np.asarray(x).reshape(-1, W.shape[0]).shape[0]
    if rounds_weight(M, dtype):
        return (O.gemv_union_rounded_f64(x, W, s, t, b, gs, dtype) if graded
                else O.dense_prefill_f64(x, W, s, gs, dtype))
    return O.gemv_union_f64(x, W, s, t, b, gs) if graded else O.dense_exact_f64(x, W, s, gs)


def dense_rounding_bound(x: np.ndarray, W: np.ndarray, scale: np.ndarray, dtype: str, group_size: int = 128):
    """Largest difference the reference's own elementwise rounding of W*s to
    the activation dtype (grinqh/kernel.py:586) can make to a dense product:
    u * (|x| @ |W*s|).  Kernels that keep W*s exact (scale applied in fp32)
    may differ from the reference's dense output by up to this much."""
    u = UNIT_ROUNDOFF[dtype]
    s = np.repeat(np.abs(np.asarray(scale, dtype=np.float64)), group_size, axis=0)[: W.shape[0]]
    return u * (np.abs(np.asarray(x, dtype=np.float64)) @ (np.abs(W.astype(np.float64)) * s))


def output_tolerance(ref_pre: np.ndarray, dtype: str, bias=None) -> np.ndarray:
    """Allowed |y - y_ref| for a kernel output against the float64 oracle.

    ``ref_pre`` is the oracle's float64 product before the output cast.  The
    kernel output carries two roundings in the output dtype (cast, then bias
    add, as in grinqh/kernel.py:706-708) -- up to 2 units of roundoff of the
    result each -- plus fp32 accumulation-order differences, bounded here by
    2e-3 of the product's rms (the tolerance stated for this path).
    """
    u = UNIT_ROUNDOFF[dtype]
    ref = np.asarray(ref_pre, dtype=np.float64)
    rms = float(np.sqrt(np.mean(ref[np.isfinite(ref)] ** 2))) if np.isfinite(ref).any() else 0.0
    mag = np.abs(ref)
    if bias is not None:
        mag = mag + np.abs(ref + np.asarray(bias, dtype=np.float64)[None, :])
    return 2.0 * u * mag + 2e-3 * rms + 1e-30


def assert_output_close(y: torch.Tensor, ref_pre: np.ndarray, ref_final: np.ndarray, dtype: str, bias=None,
                        what: str = "", extra_tol=None) -> dict:
    """Check a kernel output against the oracle and report max abs / rel error."""
    got = y.detach().float().cpu().double().numpy().reshape(ref_final.shape)
    tol = output_tolerance(ref_pre.reshape(ref_final.shape), dtype, bias)
    if extra_tol is not None:
        tol = tol + np.asarray(extra_tol).reshape(ref_final.shape)
    err = np.abs(got - ref_final)
    nan_ref = np.isnan(ref_final)
    assert np.array_equal(np.isnan(got), nan_ref), f"{what}: NaN pattern differs"
    ok = ~nan_ref
    bad = err[ok] > tol[ok]
    rel = err[ok] / np.maximum(np.abs(ref_final[ok]), 1e-30)
    stats = {"max_abs": float(err[ok].max()) if ok.any() else 0.0,
             "max_rel": float(rel.max()) if ok.any() else 0.0}
    assert not bad.any(), (f"{what}: {int(bad.sum())} of {bad.size} outputs outside tolerance; "
                           f"max abs err {stats['max_abs']:.3e}, worst excess "
                           f"{float((err[ok] - tol[ok]).max()):.3e}")
    return stats


def error_stats(y, ref_final: np.ndarray) -> dict:
    """Max abs error, max rel error (outputs with |ref| >= 1 % of rms(ref)) and
    max abs error / rms(ref) of a kernel output against a reference output."""
    got = (y.detach().float().cpu().double().numpy() if isinstance(y, torch.Tensor) else np.asarray(y, np.float64))
    ref = np.asarray(ref_final, dtype=np.float64)
    got = got.reshape(ref.shape)
    ok = np.isfinite(ref)
    if not ok.any():
        return {"max_abs": 0.0, "max_rel": 0.0, "max_abs_over_rms": 0.0, "rms": 0.0}
    err = np.abs(got[ok] - ref[ok])
    r = np.abs(ref[ok])
    rms = float(np.sqrt(np.mean(r ** 2)))
    big = r >= 0.01 * rms
    return {"max_abs": float(err.max()),
            "max_rel": float((err[big] / r[big]).max()) if big.any() else 0.0,
            "max_abs_over_rms": float(err.max() / rms) if rms > 0 else 0.0,
            "rms": rms}


def record_errors(config: str, case: str, **fields) -> None:
    """Append one error record (JSON line) to the file named by the
    GRINQH_PARITY_LOG environment variable, if set (one JSON object per line:
    config, case and the error fields)."""
    path = os.environ.get("GRINQH_PARITY_LOG")
    if not path:
        return
    os.makedirs(os.path.dirname(os.path.abspath(path)), exist_ok=True)
    with open(path, "a") as f:
        f.write(json.dumps({"config": config, "case": case, **fields}) + "\n")
