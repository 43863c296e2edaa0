"""CPU tests of the threshold-file tooling (grinqh/thresholds.py): the file
format the plugin reads through GRINQH_JSON_PATH (reference
grinqh/grinqh.py:84-92), validation against what get_quant_method needs
(:101-112), and thresholds derived from recorded activation statistics."""
import json
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
try:
    import vllm  # noqa: F401
except ImportError:
    sys.path.insert(0, os.path.join(HERE, "vllm_shim"))

from grinqh import thresholds as T  # noqa: E402
from oracle import grinqh_oracle as O  # noqa: E402


def test_llama_prefixes():
    p = T.llama_prefixes(32)
    assert len(p) == 128 and p[0] == "model.layers.0.self_attn.qkv_proj"
    assert p[-1] == "model.layers.31.mlp.down_proj" and len(set(p)) == 128


def test_save_load_roundtrip_and_plugin_reads_it(tmp_path, monkeypatch):
    """A file written by save() is what GRINQHConfig.from_config reads through
    GRINQH_JSON_PATH, and get_quant_method pads each entry to four values."""
    import grinqh
    grinqh.register()
    from grinqh.grinqh import GRINQHConfig
    from vllm.model_executor.layers.linear import LinearBase
    th = {pfx: [0.0, 0.5 + i, 1.0 + i] for i, pfx in enumerate(T.llama_prefixes(2))}
    path = str(tmp_path / "t.json")
    T.save(path, th)
    assert json.load(open(path)) == {"thresholds": {k: [float(v) for v in vals] for k, vals in th.items()}}
    assert T.load(path) == th
    monkeypatch.setenv("GRINQH_JSON_PATH", path)
    cfg = GRINQHConfig.from_config({"config_groups": {"group_0": {"weights": {"num_bits": 8, "group_size": 128}}},
                                    "grinqh": {}})
    m = cfg.get_quant_method(LinearBase(), "model.layers.1.mlp.down_proj")
    assert m.layer_thresholds == [0.0, 1.5 + 6, 2.0 + 6, 0.0]


def test_validate_errors_and_warnings():
    with pytest.raises(T.ThresholdError):
        T.validate([1, 2])
    with pytest.raises(T.ThresholdError):
        T.validate({"a": "0.5"})
    with pytest.raises(T.ThresholdError):
        T.validate({"a": [0.1, float("nan")]})
    with pytest.raises(T.ThresholdError, match="no thresholds"):
        T.validate({"model.layers.0.self_attn.qkv_proj": [0.1]}, T.llama_prefixes(1))
    w = T.validate({"a": [0.0, 1.0, 0.5, 2.0, 9.0], "b": [0.1], "c": [-1, -1, -1, -1]}, max_bits=8)
    assert any("only the first four" in s for s in w)
    assert any("a: thresholds decrease" in s for s in w)
    assert any("b: 1 values" in s for s in w)
    assert not any(s.startswith("c:") for s in w)
    with pytest.raises(T.ThresholdError):
        T.save("/dev/null", {"a": [True]})


def test_thresholds_from_statistics_give_the_requested_grade_mix():
    """Thresholds at P50/P80/P95 of the recorded statistic (zone 0 at 0.0)
    grade 50/30/15/5 % of rows to 1/2/3/4 planes under the plugin's grading
    rule (the oracle's S6, strict fp32 comparison)."""
    rng = np.random.default_rng(0)
    rec = T.StatsRecorder()
    xs = [torch.from_numpy(rng.standard_normal((16, 4096)).astype(np.float32)).half() for _ in range(8)]
    for x in xs:
        rec.update("l", x)
    s = rec.samples("l")
    assert s.shape == (8 * 4096,)
    np.testing.assert_array_equal(s[:4096], xs[0].abs().float().amax(0).numpy())
    th = T.thresholds_from_statistics({"l": s})["l"]
    assert th[0] == 0.0 and len(th) == 4
    planes = np.array([bin(int(b)).count("1") for b in O.grade(s, th, 8)])
    mix = np.bincount(planes, minlength=5)[1:] / planes.size
    np.testing.assert_allclose(mix, [0.5, 0.3, 0.15, 0.05], atol=2e-3)
    th2 = T.thresholds_from_statistics({"l": s}, (0.2, 0.4, 0.6, 0.8), first=None)["l"]
    assert len(th2) == 4 and th2[0] > 0


def test_command_line(tmp_path):
    rec = T.StatsRecorder()
    rng = np.random.default_rng(1)
    for pfx in T.llama_prefixes(1):
        rec.update(pfx, rng.standard_normal((4, 256)).astype(np.float32))
    stats = str(tmp_path / "s.npz")
    rec.save_npz(stats)
    out = str(tmp_path / "t.json")
    env = dict(os.environ, PYTHONPATH=os.path.join(os.path.dirname(HERE), "vllm-grinqh-plugin_amd"))
    r = subprocess.run([sys.executable, "-m", "grinqh.thresholds", "from-stats", stats, out], capture_output=True,
                       text=True, env=env)
    assert r.returncode == 0, r.stderr
    r = subprocess.run([sys.executable, "-m", "grinqh.thresholds", "validate", out, "--llama-layers", "1"],
                       capture_output=True, text=True, env=env)
    assert r.returncode == 0 and "ok: 4 layers" in r.stdout, r.stdout + r.stderr
    r = subprocess.run([sys.executable, "-m", "grinqh.thresholds", "validate", out, "--llama-layers", "2"],
                       capture_output=True, text=True, env=env)
    assert r.returncode != 0 and "no thresholds" in r.stderr
