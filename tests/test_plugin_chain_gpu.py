"""The plugin's whole load-and-run chain on the GPU (reference
grinqh/grinqh.py:116-247): create_weights -> the checkpoint weight loader
(int32-packed compressed-tensors shards merged into one q/k/v or gate/up
parameter; raw int8 at 6 bits) -> process_weights_after_loading (the repack on
the device) -> apply, against the float64 oracle built from the checkpoint's
own int8 weights and scales.  Without a vLLM install the layer classes come
from tests/vllm_shim, as in tests/test_plugin_surface.py.
"""
import importlib
import os

import numpy as np
import pytest
import torch

from oracle import grinqh_oracle as O
from tests._helpers import assert_output_close, dense_rounding_bound, error_stats, record_errors

import vllm  # noqa: F401  (the real vLLM, or the stand-in tests/conftest.py put on the path)

pytestmark = pytest.mark.gpu

K, GS = 512, 128
MERGED = {"qkv": (["q", "k", "v"], [256, 128, 128]), "gate_up": (["gate", "up"], [512, 512])}


@pytest.fixture(scope="module")
def gq():
    if not torch.cuda.is_available():
        pytest.fail("GPU tests need a HIP device")
    import grinqh
    grinqh.register()
    return importlib.import_module("grinqh.grinqh")


def _load_layer(gq, bits, layer_kind, thresholds, seed):
    """Build a layer through the plugin's surface and load a synthetic
    checkpoint into it shard by shard; returns the layer, its method and the
    logical int8 W [K, N] and scales [K/gs, N] the checkpoint holds."""
    from grinqh.checkpoint import pack_to_int32
    from vllm.model_executor.layers.linear import LinearBase
    shard_ids, parts = MERGED[layer_kind]
    cfg = gq.GRINQHConfig(thresholds={"model.layers.0." + layer_kind: thresholds}, max_bits=bits)
    layer = LinearBase()
    method = cfg.get_quant_method(layer, "model.layers.0." + layer_kind)
    with torch.device("cuda"):
        method.create_weights(layer, K, parts, K, sum(parts), torch.float16)
    param = getattr(layer, layer.grinqh_weight_param_name)
    g = torch.Generator().manual_seed(seed)
    lim = 1 << (bits - 1)
    ws, ss = [], []
    for sid, n in zip(shard_ids, parts):
        w_out_in = torch.randint(-lim, lim, (n, K), generator=g, dtype=torch.int32).to(torch.int8)
        s_out = (0.05 * torch.randn(n, K // GS, generator=g)).half()
        ck = w_out_in if bits == 6 else pack_to_int32(w_out_in, bits)  # checkpoint tensors arrive on the host
        param.weight_loader(param, ck, sid)
        layer.weight_scale.weight_loader(layer.weight_scale, s_out, sid)
        ws.append(w_out_in.T)
        ss.append(s_out.T)
    method.process_weights_after_loading(layer)
    W = torch.cat(ws, 1).numpy()
    s = torch.cat(ss, 1).double().numpy()
    return layer, method, W, s


@pytest.mark.parametrize("bits", [4, 6, 8])
@pytest.mark.parametrize("layer_kind", ["qkv", "gate_up"])
def test_load_repack_apply_graded_gemv_with_bias(gq, layer_kind, bits):
    """One row: the graded GEMV (S8) with a bias, through apply()."""
    rng = np.random.default_rng(bits)
    x = O.rne_cast(rng.standard_normal((1, K)), "float16")
    t = [0.0] + np.quantile(np.abs(x), [0.5, 0.8, 0.95]).tolist()
    layer, method, W, s = _load_layer(gq, bits, layer_kind, t, seed=bits)
    N = W.shape[1]
    assert layer.original_n == N // 4
    bias = O.rne_cast(rng.standard_normal(N), "float16")
    y = method.apply(layer, torch.from_numpy(x).half().cuda(), torch.from_numpy(bias).half().cuda())
    assert y.shape == (1, N) and y.dtype == torch.float16
    pre = O.gemv_f64(x, W, s, t, bits, GS)
    fin = O.gemv(x, W, s, bias, t, bits, GS, "float16")
    assert_output_close(y, pre, fin, "float16", bias=bias, what=f"{layer_kind} b={bits} graded GEMV")
    record_errors("plugin chain (loader -> repack -> apply)", f"{layer_kind} b={bits} M=1 graded, bias",
                  vs_reference=error_stats(y, fin))


@pytest.mark.parametrize("bits", [4, 6, 8])
@pytest.mark.parametrize("layer_kind", ["qkv", "gate_up"])
def test_load_repack_apply_reference_dispatch_batch(gq, layer_kind, bits):
    """Sixteen rows in the reference's dispatch (dense S9 regardless of
    thresholds, grinqh/kernel.py:663-680), with a bias, through apply().  The
    16-row kernel keeps W*s exact, so it is held to the exact dense product
    and to S9 within S9's own rounding of W*s."""
    from grinqh.kernel import batch_grading_mode
    if batch_grading_mode() != "reference":
        pytest.skip("GRINQH_BATCH_GRADING is not the reference dispatch")
    rng = np.random.default_rng(10 + bits)
    x = O.rne_cast(rng.standard_normal((16, K)), "float16")
    layer, method, W, s = _load_layer(gq, bits, layer_kind, [5.0] * 4, seed=10 + bits)
    N = W.shape[1]
    bias = O.rne_cast(rng.standard_normal(N), "float16")
    y = method.apply(layer, torch.from_numpy(x).half().cuda().view(2, 8, K), torch.from_numpy(bias).half().cuda())
    assert y.shape == (2, 8, N)
    y = y.view(16, N)
    own = O.dense_exact_f64(x, W, s, GS)
    assert_output_close(y, own, O.bias_add(own, bias, "float16"), "float16", bias=bias,
                        what=f"{layer_kind} b={bits} dense batch")
    pre = O.dense_prefill_f64(x, W, s, GS, "float16")
    fin = O.dense_prefill(x, W, s, bias, GS, "float16")
    assert_output_close(y, pre, fin, "float16", bias=bias, what=f"{layer_kind} b={bits} dense batch vs S9",
                        extra_tol=dense_rounding_bound(x, W, s, "float16"))
    record_errors("plugin chain (loader -> repack -> apply)", f"{layer_kind} b={bits} M=16 reference dispatch, bias",
                  vs_reference=error_stats(y, fin))
