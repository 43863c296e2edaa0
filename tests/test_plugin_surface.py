"""CPU tests of the plugin's vLLM surface (reference grinqh/grinqh.py and
grinqh/__init__.py): registration, config parsing, threshold lookup, parameter
creation and the checkpoint weight loader.  Without a vLLM install they run
against tests/vllm_shim; with one they run against the real vLLM.

The GPU steps (repack, apply) must refuse CPU tensors instead of computing
anything: there is no CPU fallback in the product.
"""
import importlib
import json
import os

import pytest
import torch

import vllm  # the real vLLM, or the stand-in tests/conftest.py put on the path

HERE = os.path.dirname(os.path.abspath(__file__))
REAL_VLLM = not os.path.abspath(vllm.__file__).startswith(os.path.join(HERE, "vllm_shim") + os.sep)


@pytest.fixture(scope="module")
def gq():
    import grinqh
    grinqh.register()
    return importlib.import_module("grinqh.grinqh")


def _cfg(**grinqh_cfg):
    return {"config_groups": {"group_0": {"weights": {"num_bits": 8, "group_size": 128}}}, "grinqh": grinqh_cfg}


def test_entry_point_declared():
    try:
        import tomllib
    except ImportError:  # Python 3.10
        import tomli as tomllib
    with open(os.path.join(os.path.dirname(HERE), "vllm-grinqh-plugin_amd", "pyproject.toml"), "rb") as f:
        proj = tomllib.load(f)
    assert proj["project"]["entry-points"]["vllm.general_plugins"] == {"grinqh": "grinqh:register"}


@pytest.mark.skipif(REAL_VLLM, reason="registry introspection uses the shim")
def test_register_adds_quantization_config(gq):
    from vllm.model_executor.layers.quantization import QUANTIZATION_METHODS
    assert QUANTIZATION_METHODS["grinqh"] is gq.GRINQHConfig


def test_op_schema_matches_reference(gq):
    schema = str(torch.ops.grinqh.gemm_or_gemv.default._schema)
    assert schema == ("grinqh::gemm_or_gemv(Tensor x, Tensor weight_packed, Tensor weight_scale, Tensor? bias, "
                      "SymInt max_bits, SymInt group_size, SymInt original_n, float[] thresholds, "
                      "bool use_marlin=False) -> Tensor")


def test_fake_impl_shape(gq):
    from torch._subclasses.fake_tensor import FakeTensorMode
    with FakeTensorMode():
        x = torch.empty(2, 3, 256, dtype=torch.float16)
        w = torch.empty(256, 64, dtype=torch.uint32)
        s = torch.empty(2, 256, dtype=torch.float16)
        y = torch.ops.grinqh.gemm_or_gemv(x, w, s, None, 8, 128, 64, [0.0] * 4)
    assert y.shape == (2, 3, 256) and y.dtype == torch.float16


def test_config_basics(gq):
    c = gq.GRINQHConfig.from_config(_cfg(thresholds={"a": [1.0]}))
    assert (c.get_name(), c.num_bits, c.group_size) == ("GRINQH", 8, 128)
    assert c.get_supported_act_dtypes() == [torch.float16, torch.bfloat16]
    assert gq.GRINQHConfig.get_min_capability() == 80
    assert gq.GRINQHConfig.get_config_filenames() == []
    assert gq.GRINQHConfig.override_quantization_method({}, "grinqh") == "grinqh"
    assert gq.GRINQHConfig.override_quantization_method({}, "awq") is None
    c4 = gq.GRINQHConfig.from_config({"config_groups": {"group_0": {"weights": {"num_bits": 4, "group_size": 64}}},
                                      "grinqh": {"thresholds": {}}})
    assert (c4.num_bits, c4.group_size) == (4, 64)
    c6 = gq.GRINQHConfig.from_config(_cfg(max_bits=6, thresholds={}))
    assert c6.num_bits == 6


def test_threshold_precedence(gq, tmp_path, monkeypatch):
    monkeypatch.delenv("GRINQH_JSON_PATH", raising=False)
    with pytest.raises(ValueError, match="thresholds"):
        gq.GRINQHConfig.from_config(_cfg())
    p = tmp_path / "t.json"
    p.write_text(json.dumps({"thresholds": {"model.layers.0.mlp.down_proj": [0.5, 1.0]}}))
    monkeypatch.setenv("GRINQH_JSON_PATH", str(p))
    c = gq.GRINQHConfig.from_config(_cfg(thresholds={"other": [9.0]}))
    assert c.thresholds == {"model.layers.0.mlp.down_proj": [0.5, 1.0]}


def test_get_quant_method_lookup_and_padding(gq):
    from vllm.model_executor.layers.linear import LinearBase
    c = gq.GRINQHConfig(thresholds={"m.qkv_proj": [0.1, 0.2], "m.o_proj": [1, 2, 3, 4, 5]})
    m = c.get_quant_method(LinearBase(), "m.qkv_proj")
    assert isinstance(m, gq.GRINQHLinearMethod)
    assert m.layer_thresholds == [0.1, 0.2, 0.0, 0.0] and m.layer_name == "m.qkv_proj"
    assert c.get_quant_method(LinearBase(), "m.o_proj").layer_thresholds == [1, 2, 3, 4]
    with pytest.raises(ValueError, match="no thresholds"):
        c.get_quant_method(LinearBase(), "m.gate_up_proj")
    assert c.get_quant_method(torch.nn.Module(), "m.embed") is None


def _layer(gq, bits, parts, K=256, tp=1):
    from vllm.model_executor.layers.linear import LinearBase
    cfg = gq.GRINQHConfig(thresholds={"l": [0.0] * 4}, max_bits=bits)
    layer = LinearBase(tp_size=tp)
    method = cfg.get_quant_method(layer, "l")
    method.create_weights(layer, K, parts, K, sum(parts), torch.float16)
    return layer, method


@pytest.mark.parametrize("bits", [2, 4, 6, 8])
def test_create_weights(gq, bits):
    layer, _ = _layer(gq, bits, [128, 64, 64])
    name = "weight" if bits == 6 else "weight_packed"
    assert layer.grinqh_weight_param_name == name
    w = getattr(layer, name)
    assert w.shape == (256, 64) and w.dtype == torch.int32
    assert (w.input_dim, w.output_dim, w.packed_dim, w.packed_factor) == (0, 1, 1, 4)
    assert layer.weight_scale.shape == (2, 256) and layer.weight_scale.dtype == torch.float16
    assert layer.weight_shape.shape == (2,)


def test_tensor_parallel_rejected(gq):
    with pytest.raises(NotImplementedError):
        _layer(gq, 8, [256], tp=2)


@pytest.mark.parametrize("bits", [4, 6, 8])
def test_weight_loader_merged_shards(gq, bits):
    """Loader of reference grinqh/grinqh.py:134-168: per-shard column slices of
    the int8 [K, N] weight (viewed as int32) and of the transposed scales."""
    from grinqh.checkpoint import pack_to_int32
    g = torch.Generator().manual_seed(bits)
    parts = [128, 64, 64]
    layer, _ = _layer(gq, bits, parts)
    name = layer.grinqh_weight_param_name
    param = getattr(layer, name)
    lim = 1 << (bits - 1)
    full_w, full_s = [], []
    for sid, n in zip(["q", "k", "v"], parts):
        w_out_in = torch.randint(-lim, lim, (n, 256), generator=g, dtype=torch.int32).to(torch.int8)  # [N_i, K]
        s_out = torch.randn(n, 2, generator=g).half()  # checkpoint scales are [N_i, K/gs]
        ck = w_out_in if bits == 6 else pack_to_int32(w_out_in, bits)
        param.weight_loader(param, ck, sid)
        layer.weight_scale.weight_loader(layer.weight_scale, s_out, sid)
        full_w.append(w_out_in.T)
        full_s.append(s_out.T)
    assert torch.equal(param.data.view(torch.int8), torch.cat(full_w, 1))
    assert torch.equal(layer.weight_scale.data, torch.cat(full_s, 1))
    with pytest.raises(ValueError, match="shard_id"):
        param.weight_loader(param, torch.zeros(64, 256, dtype=torch.int8), "x")


def test_checkpoint_unpack_known_answers():
    """Words derived by hand from compressed-tensors' published int32 packing
    (field i of a word holds element i of its group at bits num_bits*i, values
    stored offset by 2^(num_bits-1), trailing padding dropped), not from the
    packer in grinqh/checkpoint.py: a big-endian field order or a two's
    complement reading would fail them."""
    from grinqh.checkpoint import unpack_from_int32
    # 4 bits: values -8 -7 0 7 1 -1 3 -4 -> fields 0 1 8 15 9 7 11 4 -> 0x4B79F810
    w4 = torch.tensor([[0x4B79F810]], dtype=torch.int32)
    assert unpack_from_int32(w4, 4, (1, 8)).tolist() == [[-8, -7, 0, 7, 1, -1, 3, -4]]
    # 8 bits: -128 127 0 -1 -> fields 0 255 128 127 -> 0x7F80FF00
    w8 = torch.tensor([[0x7F80FF00]], dtype=torch.int32)
    assert unpack_from_int32(w8, 8, (1, 4)).tolist() == [[-128, 127, 0, -1]]
    # 2 bits: (-2 -1 0 1) x 4 -> fields 0 1 2 3 per byte -> 0xE4E4E4E4, a negative int32
    w2 = torch.tensor([[0xE4E4E4E4 - (1 << 32)]], dtype=torch.int32)
    assert unpack_from_int32(w2, 2, (1, 16)).tolist() == [[-2, -1, 0, 1] * 4]
    # padding: 5 of 8 fields used (3 -5 0 7 -8 -> 0xF83B); the top 3 fields hold junk and are dropped
    wp = torch.tensor([[0xF83B | (0x5A5 << 20)]], dtype=torch.int32)
    assert unpack_from_int32(wp, 4, (1, 5)).tolist() == [[3, -5, 0, 7, -8]]


def test_checkpoint_unpack_roundtrip():
    from grinqh.checkpoint import pack_to_int32, unpack_from_int32
    g = torch.Generator().manual_seed(3)
    for bits in (2, 4, 8):
        v = torch.randint(-(1 << (bits - 1)), 1 << (bits - 1), (7, 100), generator=g).to(torch.int8)
        packed = pack_to_int32(v, bits)
        assert packed.dtype == torch.int32 and packed.shape == (7, -(-100 // (32 // bits)))
        assert torch.equal(unpack_from_int32(packed, bits, (7, 100)), v)


def test_gpu_steps_refuse_cpu_tensors(gq):
    layer, method = _layer(gq, 8, [256])
    layer.weight_packed.data.zero_()
    with pytest.raises(ValueError, match="no CPU path"):
        method.process_weights_after_loading(layer)
    layer.original_n = 64
    layer.grinqh_use_marlin = False
    with pytest.raises(ValueError, match="no CPU path"):
        method.apply(layer, torch.zeros(1, 256, dtype=torch.float16))
