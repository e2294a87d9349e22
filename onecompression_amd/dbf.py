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


def _part_index(shard_id: Any) -> int:
    """Which part of a fused DBF module a loader call fills: the whole parameter (None), a part
    number, or the q/k/v letter of a fused qkv_proj."""
    if shard_id is None or isinstance(shard_id, int):
        return shard_id or 0
    if not isinstance(shard_id, str):
        raise TypeError(f"shard id must be None, an int or one of 'q', 'k', 'v'; got {type(shard_id)}")
    letters = ("q", "k", "v")
    if shard_id not in letters:
        raise ValueError(f"Unknown shard id: {shard_id}")
    return letters.index(shard_id)


def _tp_size() -> int:
    if not HAS_VLLM:
        return 1
    try:  # pragma: no cover - needs vLLM
        from vllm.distributed import get_tensor_model_parallel_world_size

        return get_tensor_model_parallel_world_size()
    except Exception:  # noqa: BLE001
        return 1


def _starts(sizes: List[int]) -> List[int]:
    """Start of each part when the parts lie back to back."""
    return [sum(sizes[:i]) for i in range(len(sizes))]


class DBFLinearMethod(LinearMethodBase):
    """DBF linear method (vllm_plugins/dbf/vllm_plugin.py:86-418)."""

    def __init__(self, quant_config: "DbfConfig"):
        self.quant_config = quant_config

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs):
        if _tp_size() != 1:
            raise ValueError("DBF layers run unsharded: tensor_parallel_size=1 is required.")
        K = input_size
        outs = list(output_partition_sizes)
        n_parts = len(outs)
        mod_cfg = getattr(layer, "_dbf_mod_cfg", None)
        if mod_cfg is None:
            logger.warning("layer %s carries no DBF module config; assuming 1.0 bit per weight",
                           getattr(layer, "prefix", "?"))
        bits = 1.0 if mod_cfg is None else mod_cfg.get("bits", 0)
        # per part p: rank r_p, and the bytes of its two packed sign factors (r_p x K and N_p x r_p)
        ranks = [compute_mid_features(bits, K, n) for n in outs]
        s2_bytes = [(r * K + 7) // 8 for r in ranks]
        s1_bytes = [(n * r + 7) // 8 for n, r in zip(outs, ranks)]
        layer._dbf_meta = {
            "part_count": n_parts, "in_features": K, "out_sizes": outs, "mid_sizes": ranks,
            "scaling2_offsets": _starts(ranks), "scaling4_offsets": _starts(outs),
            "bp1_offsets": _starts(s2_bytes), "bp3_offsets": _starts(s1_bytes),
            "bp1_sizes": s2_bytes, "bp3_sizes": s1_bytes,
        }
        attrs = {k: v for k, v in extra_weight_attrs.items() if k != "weight_loader"}

        # Checkpoint parameters: name -> (storage, per-part sizes along dim 0, or None for scaling0,
        # which holds one row per part when the module is fused).
        stacked_s0 = n_parts > 1
        params = {
            "scaling0": (torch.empty((n_parts, K) if stacked_s0 else (K,), dtype=torch.float16), None),
            "scaling2": (torch.empty(sum(ranks), dtype=torch.float16), ranks),
            "scaling4": (torch.empty(sum(outs), dtype=torch.float16), outs),
            "bp1": (torch.empty(sum(s2_bytes), dtype=torch.uint8), s2_bytes),
            "bp3": (torch.empty(sum(s1_bytes), dtype=torch.uint8), s1_bytes),
        }

        def loader_for(name: str, sizes: Optional[List[int]]):
            starts = None if sizes is None else _starts(sizes)

            def load(param: Parameter, loaded_weight: torch.Tensor, shard_id: Any = None):
                if shard_id is None and n_parts > 1:
                    raise ValueError(f"DBF parameter {name} of a fused module is loaded per part; "
                                     f"a shard_id is required.")
                p = _part_index(shard_id)
                if sizes is None:  # scaling0: its row of the stack, or the whole vector
                    (param.data[p] if stacked_s0 else param.data).copy_(loaded_weight)
                else:
                    param.data[starts[p]:starts[p] + sizes[p]].copy_(loaded_weight)

            return load

        for name, (storage, sizes) in params.items():
            prm = Parameter(storage, requires_grad=False)
            set_weight_attrs(prm, {**attrs, "weight_loader": loader_for(name, sizes)})
            layer.register_parameter(name, prm)

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
