"""DBF quantization config and linear method backed by the HIP sign kernels.

Drop-in for vllm_plugins/dbf (registered as ``"dbf"``):

- :class:`DbfConfig` keeps the reference's parsing and per-module dispatch
  (vllm_plugins/dbf/vllm_plugin.py:421-523): bits 0 or no entry ->
  unquantized, ``method`` other than ``dbf`` -> unquantized with a warning,
  fused modules whose constituents differ -> ``ValueError``; the module's
  config travels on ``layer._dbf_mod_cfg`` because create_weights has no
  prefix argument.
- :class:`DBFLinearMethod` registers ``scaling0`` ([K] or [parts, K] fp16),
  ``scaling2`` [sum r], ``scaling4`` [sum N], ``bp1`` / ``bp3`` (uint8 packed
  signs, per-part byte offsets) with per-part weight loaders and the
  ``_dbf_meta`` dict exactly as vllm_plugin.py:90-230 does; the rank is
  ``min(min(K, N), int(bits*K*N/(K+N)))`` (vllm_plugin.py:81-83).
  ``process_weights_after_loading`` repacks every part's signs once;
  ``apply`` runs two C-ABI sign matmuls per part and adds the bias.

Deviation kept on purpose: there is no process-wide fallback to a naive
torch path (vllm_plugin.py:35-56, :403-412).  A kernel error propagates, the
same way the reference propagates out-of-memory errors.
"""

from __future__ import annotations

import logging
from typing import Any, List, Optional

import torch
from torch.nn import Parameter

from . import dbf_ops
from .module_utils import lookup_module_config, parse_layer_and_module, validate_quant_config_within_shard
from .rotation import RotationMetadata, maybe_wrap_rotation_method
from .vllm_compat import (
    HAS_VLLM,
    LinearBase,
    LinearMethodBase,
    QuantizationConfig,
    UnquantizedLinearMethod,
    register_quantization_config,
    set_weight_attrs,
)

logger = logging.getLogger(__name__)


def compute_mid_features(w_bit: float, in_features: int, out_features: int) -> int:
    """DBF rank (vllm_plugin.py:81-83): int() truncation, capped at min(K, N)."""
    mid = int(w_bit * (in_features * out_features) / (in_features + out_features))
    return min(min(in_features, out_features), mid)


def _shard_id_to_index(shard_id: Any) -> int:
    if shard_id is None:
        return 0
    if isinstance(shard_id, int):
        return shard_id
    if isinstance(shard_id, str):
        mapping = {"q": 0, "k": 1, "v": 2}
        if shard_id not in mapping:
            raise ValueError(f"Unknown shard id: {shard_id}")
        return mapping[shard_id]
    raise TypeError(f"Unsupported shard id type: {type(shard_id)}")


def _tp_size() -> int:
    if not HAS_VLLM:
        return 1
    try:  # pragma: no cover - needs vLLM
        from vllm.distributed import get_tensor_model_parallel_world_size

        return get_tensor_model_parallel_world_size()
    except Exception:  # noqa: BLE001
        return 1


def _offsets(sizes: List[int]) -> List[int]:
    out, c = [], 0
    for s in sizes:
        out.append(c)
        c += s
    return out


class DBFLinearMethod(LinearMethodBase):
    """DBF linear method (vllm_plugins/dbf/vllm_plugin.py:86-418)."""

    def __init__(self, quant_config: "DbfConfig"):
        self.quant_config = quant_config

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs):
        if _tp_size() != 1:
            raise ValueError("DBF quantization currently supports only tensor_parallel_size=1.")
        del params_dtype, output_size
        part_count = len(output_partition_sizes)
        in_features = input_size
        mod_cfg = getattr(layer, "_dbf_mod_cfg", None)
        if mod_cfg is None:
            logger.warning("DBF module config is missing on layer; defaulting bits=1.0.")
            w_bit = 1.0
        else:
            w_bit = mod_cfg.get("bits", 0)
        mids = [compute_mid_features(w_bit, in_features, n) for n in output_partition_sizes]
        bp1_sizes = [(r * in_features + 7) // 8 for r in mids]
        bp3_sizes = [(n * r + 7) // 8 for n, r in zip(output_partition_sizes, mids)]
        meta = {
            "part_count": part_count,
            "in_features": in_features,
            "out_sizes": list(output_partition_sizes),
            "mid_sizes": mids,
            "scaling2_offsets": _offsets(mids),
            "scaling4_offsets": _offsets(list(output_partition_sizes)),
            "bp1_offsets": _offsets(bp1_sizes),
            "bp3_offsets": _offsets(bp3_sizes),
            "bp1_sizes": bp1_sizes,
            "bp3_sizes": bp3_sizes,
        }
        layer._dbf_meta = meta
        extra_weight_attrs = dict(extra_weight_attrs)
        extra_weight_attrs.pop("weight_loader", None)

        def make_loader(kind: str, offsets: List[int], sizes: List[int]):
            def _loader(param: Parameter, loaded_weight: torch.Tensor, shard_id: Any = None):
                idx = _shard_id_to_index(shard_id)
                if part_count > 1 and shard_id is None:
                    raise ValueError(f"DBF expects shard_id for fused module parameter {kind}.")
                if kind == "scaling0":
                    if param.data.ndim == 2:
                        param.data[idx].copy_(loaded_weight)
                    else:
                        param.data.copy_(loaded_weight)
                    return
                param.data.narrow(0, offsets[idx], sizes[idx]).copy_(loaded_weight)

            return _loader

        def reg(name, tensor, loader):
            p = Parameter(tensor, requires_grad=False)
            set_weight_attrs(p, {**extra_weight_attrs, "weight_loader": loader})
            layer.register_parameter(name, p)

        s0_shape = (part_count, in_features) if part_count > 1 else (in_features,)
        reg("scaling0", torch.empty(s0_shape, dtype=torch.float16), make_loader("scaling0", [], []))
        reg("scaling2", torch.empty(sum(mids), dtype=torch.float16),
            make_loader("scaling2", meta["scaling2_offsets"], mids))
        reg("scaling4", torch.empty(sum(output_partition_sizes), dtype=torch.float16),
            make_loader("scaling4", meta["scaling4_offsets"], list(output_partition_sizes)))
        reg("bp1", torch.empty(sum(bp1_sizes), dtype=torch.uint8),
            make_loader("bp1", meta["bp1_offsets"], bp1_sizes))
        reg("bp3", torch.empty(sum(bp3_sizes), dtype=torch.uint8),
            make_loader("bp3", meta["bp3_offsets"], bp3_sizes))

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        if getattr(layer, "_dbf_initialized", False):
            return
        meta = getattr(layer, "_dbf_meta", None)
        if meta is None:
            return
        if layer.bp1.device.type != "cuda":
            raise RuntimeError("DBFLinearMethod needs the layer on a HIP device before "
                               "process_weights_after_loading")
        parts = []
        for i in range(meta["part_count"]):
            r, n, k = meta["mid_sizes"][i], meta["out_sizes"][i], meta["in_features"]
            s0 = layer.scaling0[i] if layer.scaling0.ndim == 2 else layer.scaling0
            s2 = layer.scaling2.narrow(0, meta["scaling2_offsets"][i], r)
            s4 = layer.scaling4.narrow(0, meta["scaling4_offsets"][i], n)
            bp1 = layer.bp1.narrow(0, meta["bp1_offsets"][i], meta["bp1_sizes"][i]).contiguous()
            bp3 = layer.bp3.narrow(0, meta["bp3_offsets"][i], meta["bp3_sizes"][i]).contiguous()
            parts.append(dbf_ops.dbf_prepare(s0.data, bp1, s2.data, bp3, s4.data, k, r, n))
        layer._oc_dbf_parts = parts
        layer._dbf_initialized = True

    def apply(self, layer: torch.nn.Module, x: torch.Tensor,
              bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        if getattr(layer, "_dbf_meta", None) is None:
            raise RuntimeError("DBF meta not initialized on layer.")
        parts = getattr(layer, "_oc_dbf_parts", None)
        if parts is None:
            raise RuntimeError("DBF layer used before process_weights_after_loading")
        return dbf_ops.dbf_forward(x, parts, bias)


@register_quantization_config("dbf")
class DbfConfig(QuantizationConfig):
    """``quant_method: dbf`` (vllm_plugins/dbf/vllm_plugin.py:421-523)."""

    def __init__(self, quantization_bits: List[dict], rotation_metadata: Optional[RotationMetadata] = None):
        super().__init__()
        self.quantization_bits = quantization_bits
        self.rotation_metadata = rotation_metadata if rotation_metadata is not None else RotationMetadata()
        self._method = DBFLinearMethod(self)

    @classmethod
    def get_name(cls) -> str:
        return "dbf"

    @classmethod
    def get_supported_act_dtypes(cls) -> List[torch.dtype]:
        return [torch.bfloat16, torch.float16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 70

    @staticmethod
    def get_config_filenames() -> List[str]:
        return []

    @classmethod
    def from_config(cls, config: dict) -> "DbfConfig":
        return cls(quantization_bits=config.get("quantization_bits", []),
                   rotation_metadata=RotationMetadata.from_quant_config(config))

    def _unquantized(self, prefix):
        return maybe_wrap_rotation_method(UnquantizedLinearMethod(), prefix=prefix,
                                          metadata=self.rotation_metadata)

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        if not isinstance(layer, LinearBase):
            return None
        layer_idx, suffix = parse_layer_and_module(prefix)
        if layer_idx is None:
            return self._unquantized(prefix)
        mod_cfg = lookup_module_config(self.quantization_bits, layer_idx, suffix)
        if mod_cfg is None:
            return self._unquantized(prefix)
        if not validate_quant_config_within_shard(self.quantization_bits, layer_idx, suffix):
            raise ValueError(f"Detected some but not all shards of {prefix} are quantized. "
                             "All shards of fused layers to have the same precision.")
        bits = mod_cfg.get("bits", 0)
        method = mod_cfg.get("method", "dbf")
        if bits == 0:
            return self._unquantized(prefix)
        if method != "dbf":
            logger.warning("DBF config for %s has unsupported method=%s, falling back to "
                           "UnquantizedLinearMethod.", prefix, method)
            return self._unquantized(prefix)
        layer._dbf_prefix = prefix
        layer._dbf_mod_cfg = mod_cfg
        return maybe_wrap_rotation_method(self._method, prefix=prefix, metadata=self.rotation_metadata)


def register_vllm_plugin():
    """vLLM ``general_plugins`` entry point (vllm_plugin.py:526-528)."""
    register_quantization_config(DbfConfig)
