"""Writes the golden fixtures of this directory (``python tests/golden/make_golden.py``).

The reference ships no stored vectors (its tests draw CUDA random numbers), so
these fixtures are produced by the CPU oracle (``oracle/grinqh_oracle.py``),
whose every function is pinned independently in ``tests/test_oracle.py``.  They
freeze inputs and expected outputs so that the oracle and the HIP path are both
checked against the same bytes: plane packing and grading bit-exactly, products
through their float64 value before the output cast.

Cases (small, seeded): every bit width; the threshold sets the reference tests
use (P50/P80/P95 of the statistic, all zones via -1, no zone via the maximum,
a non-monotone set and a plugin-padded two-value set); fp16 and bf16.
"""
from __future__ import annotations

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))
from oracle import grinqh_oracle as O  # noqa: E402

K, N, GS = 256, 64, 128


def _dt(a, dtype):
    return O.rne_cast(np.asarray(a, dtype=np.float64), dtype)


def threshold_sets(sigma):
    q = np.quantile(sigma, [0.5, 0.8, 0.95]).tolist()
    return {
        "p50_p80_p95": [0.0] + q,
        "all_zones": [-1.0] * 4,
        "no_zone": [float(sigma.max())] * 4,
        "non_monotone": [q[1], 0.0, q[2], q[0]],
        "padded_two": [q[0], q[1], 0.0, 0.0],
    }


def main():
    rng = np.random.default_rng(20240601)
    for dtype in ("float16", "bfloat16"):
        for b in (2, 4, 6, 8):
            lim = 1 << (b - 1)
            W = rng.integers(-lim, lim, size=(K, N)).astype(np.int8)
            s = _dt(rng.standard_normal((K // GS, N)) * 0.02, dtype)
            out = dict(W=W, planes=O.prepare_weight(W, b), scale=s)
            for M in (1, 4):
                x = _dt(rng.standard_normal((M, K)), dtype)
                x[:, rng.permutation(K)[: K // 100 + 1]] *= 20
                x = _dt(x, dtype)
                sigma = np.abs(x).max(0).astype(np.float32)
                out[f"x_m{M}"] = x
                for name, t in threshold_sets(sigma).items():
                    bits = O.grade(sigma, t, b)
                    key = f"m{M}_{name}"
                    out[f"{key}_thresholds"] = np.asarray(t, np.float64)
                    out[f"{key}_zone_bits"] = bits.astype(np.uint8)
                    out[f"{key}_beta"] = O.midpoint_bias(bits, b).astype(np.int32)
                    out[f"{key}_y_pre"] = O.gemv_union_f64(x, W, s, t, b, GS)
                    out[f"{key}_y"] = O.gemv_union(x, W, s, None, t, b, GS, dtype)
            x = _dt(rng.standard_normal((8, K)), dtype)
            bias = _dt(rng.standard_normal(N), dtype)
            out.update(dense_x=x, dense_bias=bias, dense_y_pre=O.dense_prefill_f64(x, W, s, GS, dtype),
                       dense_y=O.dense_prefill(x, W, s, bias, GS, dtype))
            np.savez_compressed(os.path.join(HERE, f"grinqh_{dtype}_b{b}.npz"), **out)
    print(f"wrote {len([f for f in os.listdir(HERE) if f.endswith('.npz')])} fixture files to {HERE}")


if __name__ == "__main__":
    main()
