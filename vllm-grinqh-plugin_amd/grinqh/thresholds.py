"""Threshold files for GRINQH: write, validate and derive them.

The plugin reads per-layer thresholds from ``{"thresholds": {prefix: [t0, t1,
t2, t3]}}``, either in the checkpoint's ``quantization_config.grinqh`` or in
the JSON file named by ``GRINQH_JSON_PATH`` (reference grinqh/grinqh.py:84-92,
README.md:20-24).  ``prefix`` is the vLLM module name of a quantized linear
layer (``model.layers.0.self_attn.qkv_proj``; vLLM merges q/k/v and gate/up,
so those prefixes name the merged layers), and ``t_z`` is the threshold of
zone (bit-plane) z: a K-row of the weight uses plane z for a batch when
``fp32(max_m |x[m][k]|) > fp32(t_z)`` (strict; -1 turns a plane on for every
row, +inf off).  The plugin pads a shorter list with zeros and ignores
entries past the fourth (grinqh/grinqh.py:111).

Calibrating thresholds on real data is outside this package (the reference
points to a separate replication repository).  What it provides:

* ``llama_prefixes`` -- the prefixes vLLM gives a Llama-architecture model;
* ``StatsRecorder`` -- per-channel activation statistics of the inputs each
  layer sees (the union statistic sigma_k = max_m |x[m][k]| per batch);
* ``thresholds_from_statistics`` -- thresholds at chosen quantiles of those
  statistics, so that a chosen share of K-rows uses 1, 2, 3, 4 planes;
* ``validate`` / ``load`` / ``save`` -- the file format, checked the way the
  plugin will read it.

Command line::

    python -m grinqh.thresholds validate FILE [--llama-layers 32]
    python -m grinqh.thresholds from-stats STATS.npz OUT.json [--quantiles 0.5 0.8 0.95]
"""
from __future__ import annotations

import argparse
import json
import math
import sys
from typing import Dict, Iterable, List, Optional, Sequence

import numpy as np

LLAMA_LINEARS = ("self_attn.qkv_proj", "self_attn.o_proj", "mlp.gate_up_proj", "mlp.down_proj")


def llama_prefixes(num_layers: int, root: str = "model.layers") -> List[str]:
    """vLLM module names of the quantized linears of a Llama-architecture model
    (merged qkv_proj and gate_up_proj), in layer order."""
    return [f"{root}.{i}.{name}" for i in range(num_layers) for name in LLAMA_LINEARS]


class ThresholdError(ValueError):
    """A threshold file the plugin could not use."""


def validate(thresholds: Dict[str, Sequence[float]], prefixes: Optional[Iterable[str]] = None,
             max_bits: int = 8) -> List[str]:
    """Check a ``{prefix: [t0, ...]}`` mapping.  Raises ThresholdError for what
    would break the plugin (not a mapping, a value that is not a list of real
    numbers, a prefix the model needs that is missing: get_quant_method raises
    ValueError for it, grinqh/grinqh.py:105-109).  Returns warnings for what
    it accepts but probably should not get: more than four values (the extra
    ones are ignored), fewer than max_bits/2 (the rest act as 0.0, i.e. the
    plane is on for every row with a nonzero statistic), and thresholds that
    decrease with the zone (allowed: the zone sets are then not prefixes)."""
    if not isinstance(thresholds, dict):
        raise ThresholdError(f"thresholds must map layer prefixes to lists, got {type(thresholds).__name__}")
    warnings = []
    nz = max_bits // 2
    for prefix, vals in thresholds.items():
        if not isinstance(prefix, str):
            raise ThresholdError(f"layer prefix {prefix!r} is not a string")
        if not isinstance(vals, (list, tuple)) or not all(
                isinstance(v, (int, float)) and not isinstance(v, bool) for v in vals):
            raise ThresholdError(f"{prefix}: thresholds must be a list of numbers, got {vals!r}")
        if any(isinstance(v, float) and math.isnan(v) for v in vals):
            raise ThresholdError(f"{prefix}: NaN threshold (it would compare false for every row)")
        if len(vals) > 4:
            warnings.append(f"{prefix}: {len(vals)} values; only the first four are used")
        if len(vals) < nz:
            warnings.append(f"{prefix}: {len(vals)} values for {nz} planes; the missing ones act as 0.0")
        used = list(vals)[:nz]
        if any(b < a for a, b in zip(used, used[1:])):
            warnings.append(f"{prefix}: thresholds decrease with the zone {used}")
    if prefixes is not None:
        missing = [p for p in prefixes if p not in thresholds]
        if missing:
            raise ThresholdError(f"{len(missing)} layer(s) have no thresholds, e.g. {missing[:3]}")
    return warnings


def load(path: str) -> Dict[str, List[float]]:
    """The ``thresholds`` mapping of a GRINQH_JSON_PATH file, as the plugin reads it."""
    with open(path) as f:
        doc = json.load(f)
    if not isinstance(doc, dict) or "thresholds" not in doc:
        raise ThresholdError(f"{path}: expected a JSON object with a 'thresholds' key")
    validate(doc["thresholds"])
    return doc["thresholds"]


def save(path: str, thresholds: Dict[str, Sequence[float]]) -> None:
    """Write ``{"thresholds": ...}`` for GRINQH_JSON_PATH (values as floats)."""
    validate(thresholds)
    doc = {"thresholds": {k: [float(v) for v in vals] for k, vals in thresholds.items()}}
    with open(path, "w") as f:
        json.dump(doc, f, indent=1, sort_keys=True)


class StatsRecorder:
    """Per-layer activation statistics for calibration.

    ``update(prefix, x)`` records, for one batch of layer inputs ``x[..., K]``
    (a torch tensor or an array), the union statistic of every input channel,
    ``sigma_k = max_m |x[m][k]|`` in fp32 -- what the union grading compares
    with the thresholds.  ``samples(prefix)`` returns all recorded values of
    that layer (batches x channels)."""

    def __init__(self, max_batches_per_layer: int = 1024):
        self._stats: Dict[str, List[np.ndarray]] = {}
        self.max_batches = max_batches_per_layer

    def update(self, prefix: str, x) -> None:
        try:
            import torch
            if isinstance(x, torch.Tensor):
                x = x.detach().reshape(-1, x.shape[-1]).abs().float().amax(0).cpu().numpy()
            else:
                x = np.abs(np.asarray(x, dtype=np.float32).reshape(-1, np.shape(x)[-1])).max(0)
        except ImportError:  # pragma: no cover
            x = np.abs(np.asarray(x, dtype=np.float32).reshape(-1, np.shape(x)[-1])).max(0)
        lst = self._stats.setdefault(prefix, [])
        if len(lst) < self.max_batches:
            lst.append(np.asarray(x, dtype=np.float32))

    def prefixes(self) -> List[str]:
        return list(self._stats)

    def samples(self, prefix: str) -> np.ndarray:
        return np.concatenate(self._stats[prefix])

    def save_npz(self, path: str) -> None:
        np.savez_compressed(path, **{k: self.samples(k) for k in self._stats})


def thresholds_from_statistics(samples: Dict[str, np.ndarray], quantiles: Sequence[float] = (0.5, 0.8, 0.95),
                               first: Optional[float] = 0.0) -> Dict[str, List[float]]:
    """Thresholds at quantiles of each layer's recorded statistics.

    With ``first = 0.0`` (the default) zone 0 is on for every row with a
    nonzero statistic and zones 1..3 turn on above the given quantiles: the
    default (0.5, 0.8, 0.95) has about 50 / 30 / 15 / 5 % of rows use 1 / 2 /
    3 / 4 planes on statistics like the recorded ones.  With ``first = None``
    the first quantile is zone 0's threshold too (then rows below it use no
    plane at all)."""
    out = {}
    for prefix, s in samples.items():
        s = np.asarray(s, dtype=np.float64).reshape(-1)
        s = s[np.isfinite(s)]
        if s.size == 0:
            raise ThresholdError(f"{prefix}: no finite statistics recorded")
        q = [float(v) for v in np.quantile(s, list(quantiles))]
        out[prefix] = ([first] + q)[:4] if first is not None else q[:4]
    return out


def _main(argv=None) -> int:
    ap = argparse.ArgumentParser(prog="python -m grinqh.thresholds")
    sub = ap.add_subparsers(dest="cmd", required=True)
    v = sub.add_parser("validate", help="check a GRINQH_JSON_PATH file")
    v.add_argument("path")
    v.add_argument("--llama-layers", type=int, default=None,
                   help="also require every linear of a Llama model with this many layers")
    v.add_argument("--max-bits", type=int, default=8)
    f = sub.add_parser("from-stats", help="thresholds at quantiles of recorded statistics (StatsRecorder.save_npz)")
    f.add_argument("stats")
    f.add_argument("out")
    f.add_argument("--quantiles", type=float, nargs="+", default=[0.5, 0.8, 0.95])
    args = ap.parse_args(argv)
    if args.cmd == "validate":
        th = load(args.path)
        prefixes = llama_prefixes(args.llama_layers) if args.llama_layers else None
        for w in validate(th, prefixes, args.max_bits):
            print("warning:", w)
        print(f"ok: {len(th)} layers")
        return 0
    with np.load(args.stats, allow_pickle=False) as z:
        samples = {k: z[k] for k in z.files}
    th = thresholds_from_statistics(samples, args.quantiles)
    save(args.out, th)
    print(f"wrote {len(th)} layers to {args.out}")
    return 0


if __name__ == "__main__":
    sys.exit(_main())
