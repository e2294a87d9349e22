"""vLLM plugin base classes, or local stand-ins when vLLM is not installed.

When ``vllm`` is importable the real ``QuantizationConfig``,
``LinearMethodBase``, ``LinearBase``, ``UnquantizedLinearMethod``, ``FusedMoE``,
``set_weight_attrs`` and ``register_quantization_config`` are re-exported, so
the configs in this package register with a real vLLM exactly like
``vllm_plugins/gptq`` and ``vllm_plugins/dbf`` do (pyproject.toml:105-107).
Otherwise minimal stand-ins with the same method names keep the plugin
classes importable and testable (vLLM is an optional dependency here).
"""

from __future__ import annotations

from typing import Any, Dict, List, Optional

import torch
import torch.nn.functional as F

try:  # pragma: no cover - exercised only where vLLM is installed
    from vllm.model_executor.layers.linear import (  # type: ignore
        LinearBase,
        LinearMethodBase,
        UnquantizedLinearMethod,
    )
    from vllm.model_executor.layers.quantization import register_quantization_config  # type: ignore
    from vllm.model_executor.layers.quantization.base_config import (  # type: ignore
        QuantizationConfig,
        QuantizeMethodBase,
    )
    from vllm.model_executor.utils import set_weight_attrs  # type: ignore

    try:
        from vllm.model_executor.layers.fused_moe import FusedMoE  # type: ignore
    except Exception:  # noqa: BLE001
        FusedMoE = None
    try:
        from vllm.model_executor.layers.linear import WEIGHT_LOADER_V2_SUPPORTED  # type: ignore
    except Exception:  # noqa: BLE001
        WEIGHT_LOADER_V2_SUPPORTED = None
    try:
        from vllm.model_executor.layers.linear import (  # type: ignore
            register_weight_loader_v2_supported_method as _vllm_register_v2,
        )
    except Exception:  # noqa: BLE001
        _vllm_register_v2 = None

    def register_weight_loader_v2_supported_method(cls):
        """Put ``cls``'s name on vLLM's v2 weight-loader list (the registry function when the
        installed vLLM has one, else the list itself)."""
        if _vllm_register_v2 is not None:
            return _vllm_register_v2(cls)
        if WEIGHT_LOADER_V2_SUPPORTED is not None and cls.__name__ not in WEIGHT_LOADER_V2_SUPPORTED:
            WEIGHT_LOADER_V2_SUPPORTED.append(cls.__name__)
        return cls

    HAS_VLLM = True
except Exception:  # noqa: BLE001 - any import failure means "no vLLM"
    HAS_VLLM = False

    class QuantizeMethodBase:
        """Stand-in for vllm...base_config.QuantizeMethodBase."""

        def create_weights(self, layer: torch.nn.Module, *args, **kwargs):
            raise NotImplementedError

        def apply(self, layer: torch.nn.Module, *args, **kwargs) -> torch.Tensor:
            raise NotImplementedError

        def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
            return None

    class LinearMethodBase(QuantizeMethodBase):
        """Stand-in for vllm...linear.LinearMethodBase."""

    class QuantizationConfig:
        """Stand-in for vllm...base_config.QuantizationConfig."""

        def __init__(self):
            self.packed_modules_mapping: Dict[str, List[str]] = {}

        @classmethod
        def get_name(cls) -> str:
            raise NotImplementedError

        @classmethod
        def get_supported_act_dtypes(cls) -> List[torch.dtype]:
            raise NotImplementedError

        @classmethod
        def get_min_capability(cls) -> int:
            raise NotImplementedError

        @staticmethod
        def get_config_filenames() -> List[str]:
            raise NotImplementedError

        @classmethod
        def from_config(cls, config: Dict[str, Any]) -> "QuantizationConfig":
            raise NotImplementedError

        def get_quant_method(self, layer: torch.nn.Module, prefix: str):
            raise NotImplementedError

    # vLLM hands a linear layer's params the v2 weight loader when the quant method's class name
    # is on this list (LinearBase.__init__), else the v1 loader.  The names below are the vLLM
    # methods this package meets or replaces; vLLM's own GPTQ method is among them.
    WEIGHT_LOADER_V2_SUPPORTED: List[str] = [
        "UnquantizedLinearMethod", "GPTQLinearMethod", "GPTQMarlinLinearMethod", "AWQLinearMethod",
        "AWQMarlinLinearMethod", "MarlinLinearMethod", "Fp8LinearMethod", "CompressedTensorsLinearMethod",
    ]

    def register_weight_loader_v2_supported_method(cls):
        if cls.__name__ not in WEIGHT_LOADER_V2_SUPPORTED:
            WEIGHT_LOADER_V2_SUPPORTED.append(cls.__name__)
        return cls

    def _part_slot(loaded_shard_id: Any, n_parts: int) -> int:
        if isinstance(loaded_shard_id, int):
            return loaded_shard_id
        letters = ("q", "k", "v")[:n_parts]
        if loaded_shard_id not in letters:
            raise ValueError(f"unknown shard id {loaded_shard_id!r}")
        return letters.index(loaded_shard_id)

    class _V2Parameter(torch.nn.Parameter):
        """A parameter that loads itself, as vLLM's v2 parameter classes do."""

        def load_column_parallel_weight(self, loaded_weight: torch.Tensor) -> None:
            self.data.copy_(loaded_weight)

        def load_merged_column_weight(self, loaded_weight: torch.Tensor, shard_offset: int,
                                      shard_size: int) -> None:
            self.data.narrow(self.output_dim, shard_offset, shard_size).copy_(loaded_weight)

    class LinearBase(torch.nn.Module):
        """Minimal linear layer in vLLM's style: the quant method owns the params.

        ``output_partition_sizes`` lists the fused parts (e.g. q, k, v).  As in vLLM, the weight
        loader handed to ``create_weights`` is chosen by the quant method's class name: v2 when
        it is on ``WEIGHT_LOADER_V2_SUPPORTED`` (the param must then load itself), else v1
        (driven by the param's ``output_dim`` / ``packed_dim`` / ``pack_factor`` attributes).
        """

        def __init__(self, input_size: int, output_size: int, bias: bool = False,
                     params_dtype: torch.dtype = torch.float16,
                     quant_config: Optional["QuantizationConfig"] = None, prefix: str = "",
                     output_partition_sizes: Optional[List[int]] = None):
            super().__init__()
            self.input_size = input_size
            self.output_size = output_size
            self.params_dtype = params_dtype
            self.prefix = prefix
            self.output_partition_sizes = list(output_partition_sizes or [output_size])
            if quant_config is None:
                self.quant_method = UnquantizedLinearMethod()
            else:
                self.quant_method = quant_config.get_quant_method(self, prefix)
            if self.quant_method is None:
                self.quant_method = UnquantizedLinearMethod()
            v2 = self.quant_method.__class__.__name__ in WEIGHT_LOADER_V2_SUPPORTED
            self.loader_version = 2 if v2 else 1
            self.quant_method.create_weights(self, input_size, self.output_partition_sizes,
                                             input_size, output_size, params_dtype,
                                             weight_loader=self.weight_loader_v2 if v2 else self.weight_loader)
            if bias:
                self.bias = torch.nn.Parameter(torch.zeros(output_size, dtype=params_dtype),
                                               requires_grad=False)
            else:
                self.register_parameter("bias", None)

        def _shard_range(self, param, loaded_shard_id):
            """Offset and size of a fused part along the param's output dim (in packed units when
            the param is packed along it)."""
            sizes = self.output_partition_sizes
            i = _part_slot(loaded_shard_id, len(sizes))
            off, size = sum(sizes[:i]), sizes[i]
            if getattr(param, "packed_dim", None) == param.output_dim:
                off, size = off // param.pack_factor, size // param.pack_factor
            return int(off), int(size)

        def weight_loader(self, param, loaded_weight: torch.Tensor, loaded_shard_id: Any = None):
            """v1: the whole tensor, or one fused part placed along ``param.output_dim``."""
            out_dim = getattr(param, "output_dim", None)
            if loaded_shard_id is None or out_dim is None or len(self.output_partition_sizes) == 1:
                param.data.copy_(loaded_weight)
                return
            off, size = self._shard_range(param, loaded_shard_id)
            param.data.narrow(out_dim, off, size).copy_(loaded_weight)

        def weight_loader_v2(self, param, loaded_weight: torch.Tensor, loaded_shard_id: Any = None):
            """v2: the parameter loads itself (a plain Parameter has no such methods and fails)."""
            if loaded_shard_id is None or len(self.output_partition_sizes) == 1:
                param.load_column_parallel_weight(loaded_weight=loaded_weight)
                return
            off, size = self._shard_range(param, loaded_shard_id)
            param.load_merged_column_weight(loaded_weight=loaded_weight, shard_offset=off, shard_size=size)

        def forward(self, x: torch.Tensor) -> torch.Tensor:
            return self.quant_method.apply(self, x, self.bias)

    class UnquantizedLinearMethod(LinearMethodBase):
        """Stand-in for vllm...linear.UnquantizedLinearMethod (dense F.linear; v2-native params)."""

        def create_weights(self, layer, input_size_per_partition, output_partition_sizes,
                           input_size, output_size, params_dtype, **extra_weight_attrs):
            w = _V2Parameter(torch.empty(sum(output_partition_sizes), input_size_per_partition,
                                         dtype=params_dtype), requires_grad=False)
            set_weight_attrs(w, {"input_dim": 1, "output_dim": 0, **extra_weight_attrs})
            layer.register_parameter("weight", w)

        def apply(self, layer, x, bias=None):
            return F.linear(x, layer.weight, bias)

    class FusedMoE(torch.nn.Module):
        """Minimal MoE experts layer in vLLM's style: the quant method owns the expert params
        (``create_weights(layer, num_experts, hidden_size, intermediate_size_per_partition,
        params_dtype)``), the weight loader takes ``(param, loaded, weight_name, shard_id,
        expert_id)`` with shard_id ``w1`` (gate), ``w3`` (up) or ``w2`` (down), and forward
        takes the router's top-k weights and ids.  ``activation``: ``"silu"`` or
        ``"swigluoai"`` (gpt-oss)."""

        def __init__(self, num_experts: int, top_k: int, hidden_size: int, intermediate_size: int,
                     params_dtype: torch.dtype = torch.float16,
                     quant_config: Optional["QuantizationConfig"] = None, prefix: str = "",
                     activation: str = "silu", has_bias: bool = False):
            super().__init__()
            self.global_num_experts = num_experts
            self.top_k = top_k
            self.hidden_size = hidden_size
            self.intermediate_size_per_partition = intermediate_size
            self.params_dtype = params_dtype
            self.prefix = prefix
            self.activation = activation
            self.has_bias = has_bias
            self.apply_router_weight_on_input = False
            self.expert_map = None
            self.quant_method = None if quant_config is None else quant_config.get_quant_method(self, prefix)
            if self.quant_method is None:
                raise NotImplementedError("the stand-in FusedMoE serves quantized experts only")
            self.quant_method.create_weights(self, num_experts, hidden_size, intermediate_size, params_dtype,
                                             weight_loader=self.weight_loader)

        def weight_loader(self, param, loaded_weight, weight_name: str, shard_id: str, expert_id: int,
                          return_success: bool = False):
            return param.weight_loader(param, loaded_weight, weight_name, shard_id, expert_id, return_success)

        def forward(self, hidden_states: torch.Tensor, topk_weights: torch.Tensor,
                    topk_ids: torch.Tensor) -> torch.Tensor:
            return self.quant_method.apply(self, hidden_states, topk_weights, topk_ids, None)

    def set_weight_attrs(weight: torch.Tensor, weight_attrs: Optional[Dict[str, Any]]) -> None:
        if weight_attrs is None:
            return
        for key, value in weight_attrs.items():
            if hasattr(weight, key) and key != "weight_loader":
                raise AttributeError(f"Overwriting existing tensor attribute: {key}")
            setattr(weight, key, value)

    _REGISTRY: Dict[str, type] = {}

    def register_quantization_config(name_or_cls):
        """Decorator/func registering a QuantizationConfig under its name (local registry)."""

        def _reg(cls):
            _REGISTRY[cls.get_name()] = cls
            return cls

        if isinstance(name_or_cls, str):
            return _reg
        return _reg(name_or_cls)


def registered_configs() -> Dict[str, type]:
    """Quantization configs registered through the local stand-in registry."""
    if HAS_VLLM:  # pragma: no cover
        return {}
    return dict(_REGISTRY)
