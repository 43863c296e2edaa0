"""BASELINE configs[3] stand-in, held to the oracle: two Llama-3-8B decoder
layers' quantized linears at batch 32, as bench.py's llama8b_decode_step runs
them, every product checked against the float64 oracle on its own input.

The layers are built through the plugin's surface (GRINQHConfig ->
get_quant_method -> create_weights -> the checkpoint weight loader, q/k/v and
gate/up shards merged -> process_weights_after_loading -> apply), with the
thresholds the way a deployment gets them: a dense calibration pass records
every layer's input statistic (grinqh.thresholds.StatsRecorder), the
thresholds come from its quantiles (zone 0 at 0.0), they are written with
grinqh.thresholds.save, and GRINQHConfig.from_config reads them back from
GRINQH_JSON_PATH (reference grinqh/grinqh.py:76-99).  The step then runs in
the three modes the bench times -- "reference" (the reference's dispatch: the
dense product S9 for more than one row, grinqh/kernel.py:561-587), "union"
(union grading of the batch, :249-289) and "union_fused" (union grading with
the statistic emitted by the producers: RMSNorm with the residual add, and
SiLU*mul, grinqh.producer) -- with RMSNorm, residual adds and SiLU*mul in
torch and attention replaced by the query part of the qkv output.  Every
linear's output is held to the oracle on the input it actually received (so
errors do not compound), on its first and last 1024 output columns, with the
base tolerance of the kernel's own product (rounded scaled weight at 32 rows
in fp16).
"""
import importlib

import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import assert_output_close, own_product

import vllm  # noqa: F401  (the real vLLM, or the stand-in tests/conftest.py put on the path)

pytestmark = pytest.mark.gpu

H, F, BATCH, LAYERS, BITS, GS = 4096, 14336, 32, 2, 8, 128
# module: (K, shard ids, shard widths)
MODULES = {"self_attn.qkv_proj": (H, ["q", "k", "v"], [4096, 1024, 1024]),
           "self_attn.o_proj": (H, None, [H]),
           "mlp.gate_up_proj": (H, ["gate", "up"], [F, F]),
           "mlp.down_proj": (F, None, [H])}
COLS_HELD = 1024


@pytest.fixture(scope="module")
def gq():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    import grinqh
    grinqh.register()
    return importlib.import_module("grinqh.grinqh")


def _prefixes():
    from grinqh.thresholds import llama_prefixes
    return llama_prefixes(LAYERS)


@pytest.fixture(scope="module")
def model(gq):
    """Per prefix: the layer (weights loaded and repacked), the checkpoint's
    int8 W [K, N] and fp16 scales [K/gs, N] on the host."""
    from grinqh.checkpoint import pack_to_int32
    from vllm.model_executor.layers.linear import LinearBase
    provisional = gq.GRINQHConfig(thresholds={p: [-1.0] * 4 for p in _prefixes()}, max_bits=BITS, group_size=GS)
    g = torch.Generator().manual_seed(8003)
    out = {}
    for p in _prefixes():
        K, shard_ids, parts = MODULES[p.split(".", 3)[3]]
        layer = LinearBase()
        method = provisional.get_quant_method(layer, p)
        with torch.device("cuda"):
            method.create_weights(layer, K, parts, K, sum(parts), torch.float16)
        param = getattr(layer, layer.grinqh_weight_param_name)
        ws, ss = [], []
        for sid, n in zip(shard_ids or [None], parts):
            w_out_in = torch.randint(-128, 128, (n, K), generator=g, dtype=torch.int32).to(torch.int8)
            s_out = (0.0025 * torch.rand(n, K // GS, generator=g) + 0.0005).half()
            param.weight_loader(param, pack_to_int32(w_out_in, BITS), sid)
            layer.weight_scale.weight_loader(layer.weight_scale, s_out, sid)
            ws.append(w_out_in.T.numpy())
            ss.append(s_out.T.float().numpy().astype(np.float64))
        method.process_weights_after_loading(layer)
        out[p] = (layer, np.concatenate(ws, axis=1), np.concatenate(ss, axis=1))
    return out


def _run_step(model, methods, mode, record):
    """One decode step over the layers; record[prefix] = (x, y) of each linear."""
    from grinqh import kernel as gk
    from grinqh.producer import gemv_batch_union_sigma, rmsnorm_sigma, silu_mul_sigma
    norm_w = torch.ones(H, device="cuda", dtype=torch.float16)

    def rmsnorm(h):
        hf = h.float()
        return (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5)).half() * norm_w

    def linear(p, x):
        layer = model[p][0]
        y = methods[p].apply(layer, x)
        record[p] = (x, y)
        return y

    def linear_sig(p, x, sig):
        layer, m = model[p][0], methods[p]
        y = gemv_batch_union_sigma(x, getattr(layer, layer.grinqh_weight_param_name), layer.weight_scale, None,
                                   BITS, GS, layer.original_n, m.layer_thresholds, sig)
        record[p] = (x, y)
        return y

    g = torch.Generator().manual_seed(77)
    h = (torch.randn(BATCH, H, generator=g) * 0.05).half().cuda()
    saved = gk.batch_grading_mode()
    try:
        gk.set_batch_grading_mode("reference" if mode == "reference" else "union")
        if mode != "union_fused":
            for li in range(LAYERS):
                base = f"model.layers.{li}."
                qkv = linear(base + "self_attn.qkv_proj", rmsnorm(h))
                h = h + linear(base + "self_attn.o_proj", qkv[:, :H].contiguous())
                gu = linear(base + "mlp.gate_up_proj", rmsnorm(h))
                act = (torch.nn.functional.silu(gu[:, :F].float()) * gu[:, F:].float()).half()
                h = h + linear(base + "mlp.down_proj", act)
        else:
            hn, sig, res = rmsnorm_sigma(h, norm_w)
            for li in range(LAYERS):
                base = f"model.layers.{li}."
                qkv = linear_sig(base + "self_attn.qkv_proj", hn, sig)
                o = linear(base + "self_attn.o_proj", qkv[:, :H].contiguous())
                hn, sig, res = rmsnorm_sigma(o, norm_w, 1e-5, res)
                gu = linear_sig(base + "mlp.gate_up_proj", hn, sig)
                a, asig = silu_mul_sigma(gu)
                d = linear_sig(base + "mlp.down_proj", a, asig)
                hn, sig, res = rmsnorm_sigma(d, norm_w, 1e-5, res)
        torch.cuda.synchronize()
    finally:
        gk.set_batch_grading_mode(saved)


def test_decode_step_linears_against_oracle(gq, model, tmp_path, monkeypatch):
    from grinqh.thresholds import StatsRecorder, save, thresholds_from_statistics
    prefixes = _prefixes()
    # ---- calibration: a dense pass (reference dispatch, provisional thresholds)
    provisional = {p: gq.GRINQHConfig(thresholds={p: [-1.0] * 4}).get_quant_method(model[p][0], p)
                   for p in prefixes}
    rec = {}
    _run_step(model, provisional, "reference", rec)
    stats = StatsRecorder()
    for p in prefixes:
        stats.update(p, rec[p][0])
    calibrated = thresholds_from_statistics({p: stats.samples(p) for p in prefixes})
    path = tmp_path / "grinqh_thresholds.json"
    save(str(path), calibrated)
    # ---- the deployment path: thresholds from GRINQH_JSON_PATH
    monkeypatch.setenv("GRINQH_JSON_PATH", str(path))
    cfg = gq.GRINQHConfig.from_config({"config_groups": {"group_0": {"weights": {"num_bits": BITS,
                                                                                 "group_size": GS}}}})
    assert cfg.num_bits == BITS and cfg.group_size == GS
    methods = {p: cfg.get_quant_method(model[p][0], p) for p in prefixes}
    for p in prefixes:
        assert methods[p].layer_thresholds == pytest.approx(calibrated[p])
    # ---- the three modes, every linear held to the oracle on its own input
    checked = 0
    for mode in ("reference", "union", "union_fused"):
        rec = {}
        _run_step(model, methods, mode, rec)
        assert set(rec) == set(prefixes)
        for p in prefixes:
            x, y = rec[p]
            _, W, s = model[p]
            N = W.shape[1]
            cols = np.r_[0:COLS_HELD, N - COLS_HELD:N]
            xn = x.double().cpu().numpy()
            graded = mode != "reference"
            t = methods[p].layer_thresholds
            pre = own_product(xn, W[:, cols], s[:, cols], t, BITS, GS, "float16", graded)
            fin = O.bias_add(pre, None, "float16")
            ys = y[:, torch.from_numpy(cols).cuda()]
            assert_output_close(ys, pre, fin, "float16", what=f"{mode} {p}")
            if graded:  # the grading really skipped planes: not every row uses all four
                zb = O.grade(O.union_sigma(xn), t, BITS)
                assert (zb != 0b1111).any(), f"{mode} {p}: every row of K used all planes"
            checked += 1
    assert checked == 3 * len(prefixes)
