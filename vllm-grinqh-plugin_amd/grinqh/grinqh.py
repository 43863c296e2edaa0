"""vLLM integration of GRINQH: quantization config and linear method.

Same surface as the reference (grinqh/grinqh.py): ``GRINQHConfig`` registered
as ``"grinqh"``, ``GRINQHLinearMethod`` with create_weights /
process_weights_after_loading / apply, ``GRINQH_JSON_PATH`` threshold override.
The load-time repack and the forward product run on gfx950 kernels
(libgrinqh_hip.so); the Marlin fallback of the reference is gone because one
kernel family covers every bit width.
"""
from __future__ import annotations

import json
import os
from typing import List, Optional

import torch
from torch.nn.parameter import Parameter
from vllm.logger import init_logger
from vllm.model_executor import PackedvLLMParameter
from vllm.model_executor.layers.linear import LinearBase, LinearMethodBase
from vllm.model_executor.layers.quantization import register_quantization_config
from vllm.model_executor.layers.quantization.base_config import QuantizationConfig, QuantizeMethodBase
from vllm.model_executor.layers.quantization.utils import replace_parameter
from vllm.model_executor.utils import set_weight_attrs

from .checkpoint import unpack_from_int32
from .kernel import grinqh_gemm_or_gemv  # noqa: F401  (registers torch.ops.grinqh)
from .utils import prepare_weight

logger = init_logger("vllm.grinqh")
_SHARD_IDS = {"q": 0, "k": 1, "v": 2, "gate": 0, "up": 1}


def _resolve_shard_id(shard_id) -> int:
    """Merged-layer shard index (reference grinqh/grinqh.py:32-40)."""
    if shard_id is None:
        return 0
    if isinstance(shard_id, int):
        return shard_id
    if shard_id in _SHARD_IDS:
        return _SHARD_IDS[shard_id]
    raise ValueError(f"GRINQH: unsupported shard_id {shard_id!r}")


@register_quantization_config("grinqh")
class GRINQHConfig(QuantizationConfig):
    """Reference grinqh/grinqh.py:43-113."""

    def __init__(self, thresholds: dict, max_bits: int = 8, group_size: int = 128):
        super().__init__()
        self.thresholds = thresholds
        self.num_bits = max_bits
        self.group_size = group_size

    def get_name(self) -> str:
        return "GRINQH"

    def get_supported_act_dtypes(self) -> list:
        return [torch.float16, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 80

    @staticmethod
    def get_config_filenames() -> list:
        return []

    @classmethod
    def override_quantization_method(cls, hf_quant_cfg, user_quant, hf_config=None):
        if user_quant == "grinqh":
            return "grinqh"
        return None

    @classmethod
    def from_config(cls, config: dict) -> "GRINQHConfig":
        """Threshold precedence: ``GRINQH_JSON_PATH`` file, then the checkpoint's
        ``grinqh.thresholds``, else ValueError (reference grinqh/grinqh.py:76-99)."""
        group_0_weights = config.get("config_groups", {}).get("group_0", {}).get("weights", {})
        grinqh_cfg = config.get("grinqh", {})
        num_bits = grinqh_cfg.get("max_bits", group_0_weights.get("num_bits", 8))
        group_size = group_0_weights.get("group_size", 128)

        json_path = os.environ.get("GRINQH_JSON_PATH")
        if json_path is not None:
            logger.warning("GRINQH: GRINQH_JSON_PATH is set, overriding checkpoint thresholds with %s", json_path)
            with open(json_path) as f:
                thresholds = json.load(f)["thresholds"]
        elif "thresholds" in grinqh_cfg:
            thresholds = grinqh_cfg["thresholds"]
        else:
            raise ValueError(
                "GRINQH: checkpoint quantization_config has no 'grinqh.thresholds'. "
                "Calibrate the model first or set GRINQH_JSON_PATH.")
        return cls(thresholds=thresholds, max_bits=num_bits, group_size=group_size)

    def get_quant_method(self, layer: torch.nn.Module, prefix: str) -> Optional[QuantizeMethodBase]:
        if isinstance(layer, LinearBase):
            t_vals = self.thresholds.get(prefix)
            if t_vals is None:
                raise ValueError(
                    f"GRINQH: no thresholds for layer '{prefix}'. Thresholds "
                    "must be keyed by vLLM module names (e.g. qkv_proj).")
            t_vals = (list(t_vals) + [0.0] * 4)[:4]
            return GRINQHLinearMethod(self, t_vals, layer_name=prefix)
        return None


class GRINQHLinearMethod(LinearMethodBase):
    """Reference grinqh/grinqh.py:116-247."""

    def __init__(self, quant_config: GRINQHConfig, layer_thresholds: List[float] = None,
                 layer_name: str = "unknown"):
        super().__init__()
        self.quant_config = quant_config
        self.layer_thresholds = layer_thresholds
        self.layer_name = layer_name
        self.PACK_FACTOR = 4

    def create_weights(self, layer, input_size_per_partition, output_partition_sizes, input_size, output_size,
                       params_dtype, **extra_weight_attrs):
        """Parameters ``weight_packed`` (``weight`` at 6 bits) int32 ``[K, N/4]``
        holding int8 ``W[K, N]``, ``weight_scale`` ``[ceil(K/gs), N]`` and a
        dummy ``weight_shape`` (reference grinqh/grinqh.py:124-198).  Tensors go
        to the ambient default device that vLLM sets while building the model."""
        if getattr(layer, "tp_size", 1) > 1:
            raise NotImplementedError("GRINQH does not support tensor parallelism (tp_size > 1) as of now.")
        output_size_per_partition = sum(output_partition_sizes)
        scales_block_m = self.quant_config.group_size
        is_6bit = self.quant_config.num_bits == 6
        param_name = "weight" if is_6bit else "weight_packed"
        pack = self.PACK_FACTOR
        num_bits = self.quant_config.num_bits

        def grinqh_weight_loader(param, loaded_weight, shard_id=None):
            current_shard = _resolve_shard_id(shard_id)
            if param is scales:
                s = loaded_weight.to(param.device).T.contiguous()
                if s.shape == param.shape:
                    param.data.copy_(s)
                else:
                    start = sum(output_partition_sizes[:current_shard])
                    length = output_partition_sizes[current_shard]
                    param.data[:, start:start + length].copy_(s)
                return
            if is_6bit:
                w = loaded_weight.to(param.device)
            else:
                w = unpack_from_int32(loaded_weight.to(param.device), num_bits, param.T.shape)
            w = w.T.contiguous().to(torch.int8)
            if len(output_partition_sizes) > 1:
                start_packed = sum(output_partition_sizes[:current_shard]) // pack
                size_packed = output_partition_sizes[current_shard] // pack
                param.data[:, start_packed:start_packed + size_packed].copy_(w.view(torch.int32))
            else:
                param.data[:, :].copy_(w.view(torch.int32))

        weight = PackedvLLMParameter(
            data=torch.empty(input_size_per_partition, output_size_per_partition // pack, dtype=torch.int32),
            input_dim=0, output_dim=1, packed_dim=1, packed_factor=pack,
            weight_loader=grinqh_weight_loader,
        )
        layer.register_parameter(param_name, weight)
        layer.grinqh_weight_param_name = param_name

        scale_rows = (input_size_per_partition + scales_block_m - 1) // scales_block_m
        scales = Parameter(torch.empty(scale_rows, output_size_per_partition, dtype=params_dtype),
                           requires_grad=False)
        layer.register_parameter("weight_scale", scales)
        set_weight_attrs(scales, {"weight_loader": grinqh_weight_loader})

        weight_shape = Parameter(torch.empty(2, dtype=torch.int64), requires_grad=False)
        set_weight_attrs(weight_shape, {"weight_loader": lambda p, w, shard_id=None: None})
        layer.register_parameter("weight_shape", weight_shape)

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        """Repack the int8 weight into the bit-plane layout on the GPU
        (reference grinqh/grinqh.py:200-210, one fused kernel)."""
        param = getattr(layer, layer.grinqh_weight_param_name)
        w = param.data.view(torch.int8)
        layer.original_n = w.shape[1] // self.PACK_FACTOR
        packed = prepare_weight(w, self.quant_config.num_bits)
        replace_parameter(layer, layer.grinqh_weight_param_name, packed)
        layer.grinqh_use_marlin = False

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        return torch.ops.grinqh.gemm_or_gemv(
            x,
            getattr(layer, layer.grinqh_weight_param_name),
            layer.weight_scale,
            bias,
            self.quant_config.num_bits,
            self.quant_config.group_size,
            layer.original_n,
            self.layer_thresholds,
            layer.grinqh_use_marlin,
        )
