"""Mixed-GPTQ quantization config and linear method backed by the HIP kernels.

Drop-in for vllm_plugins/gptq (registered as ``"mixed_gptq"``):

- :class:`MixedGPTQConfig` keeps the reference's config parsing and per-module
  dispatch (vllm_plugins/gptq/vllm_plugin.py:83-365): ``quantization_bits``
  (or legacy ``layer_bits``), group size priority direct > ``params`` >
  global, ``desc_act``, ``sym``, ``lm_head`` and ``checkpoint_format``
  defaulting to ``"gptq_v2"`` when absent.  bits 0 or no entry -> unquantized;
  fused modules whose constituents differ -> ``ValueError``.
- Where the reference hands 4/8-bit symmetric layers to vLLM's Marlin kernel
  and everything else to vLLM's Exllama kernel (:332-353,
  vllm_plugins/gptq/constants.py:12-31), every GPTQ layer here goes to
  :class:`MixedGPTQLinearMethod`, one HIP kernel family for 2/3/4/8 bits with or
  without act-order.
- :class:`MixedGPTQLinearMethod` registers the checkpoint tensors under the same
  names and shapes (``qweight`` [K*b/32, N] int32, ``qzeros`` [G, N*b/32]
  int32, ``scales`` [G, N], ``g_idx`` [K] int32), repacks them once in
  ``process_weights_after_loading`` and runs ``apply`` as one C-ABI call.

Deviation kept on purpose: ``scales`` are stored in fp16, the checkpoint
dtype, also for bf16 models, so the dequantised weight equals OneComp's own
``RNE(fp32(s) * (q - z))`` bit for bit.
"""

from __future__ import annotations

import logging
import re
from fractions import Fraction
from typing import Any, Dict, List, Optional

import torch

from . import ops
from . import _native as N
from .module_utils import (
    constituent_configs,
    lookup_module_config,
    parse_layer_and_module,
    validate_quant_config_within_shard,
)
from .rotation import RotationMetadata, maybe_wrap_rotation_method
from .vllm_compat import (
    FusedMoE,
    LinearBase,
    LinearMethodBase,
    QuantizationConfig,
    QuantizeMethodBase,
    UnquantizedLinearMethod,
    register_quantization_config,
    set_weight_attrs,
)

logger = logging.getLogger(__name__)

SUPPORTED_BITS = (2, 3, 4, 8)
_MOE_EXPERT_CFG_RE = re.compile(r"(?:^|\.)experts\.\d+\.")


class GPTQLayerConfig:
    """Per-layer GPTQ parameters handed to :class:`MixedGPTQLinearMethod`."""

    def __init__(self, bits: int, group_size: int, desc_act: bool, sym: bool,
                 checkpoint_format: str):
        if bits not in SUPPORTED_BITS:
            raise ValueError(f"GPTQ bits must be one of {SUPPORTED_BITS}, got {bits}")
        self.weight_bits = bits
        self.group_size = group_size
        self.desc_act = desc_act
        self.sym = sym
        self.checkpoint_format = checkpoint_format
        self.pack_factor = Fraction(32, bits)

    @property
    def zero_format(self) -> int:
        return N.OC_ZERO_V2 if self.checkpoint_format == "gptq_v2" else N.OC_ZERO_V1

    def __repr__(self):
        return (f"GPTQLayerConfig(bits={self.weight_bits}, group_size={self.group_size}, "
                f"desc_act={self.desc_act}, checkpoint_format={self.checkpoint_format})")


def _shard_offsets(output_partition_sizes: List[int]):
    offs, c = [], 0
    for s in output_partition_sizes:
        offs.append(c)
        c += s
    return offs


def _shard_index(shard_id: Any, n_parts: int) -> int:
    if shard_id is None:
        return 0
    if isinstance(shard_id, int):
        return shard_id
    mapping = {"q": 0, "k": 1, "v": 2}
    if isinstance(shard_id, str) and shard_id in mapping and mapping[shard_id] < n_parts:
        return mapping[shard_id]
    raise ValueError(f"Unknown shard id: {shard_id}")


class MixedGPTQLinearMethod(LinearMethodBase):
    """Linear method for one GPTQ layer (replaces vLLM's GPTQ/Marlin methods).

    vLLM chooses a layer's weight loader by the method's class name (names in its
    WEIGHT_LOADER_V2_SUPPORTED list get the v2 loader, which needs vLLM's parameter classes).
    This method registers plain Parameters with the v1 attributes (input_dim, output_dim,
    packed_dim, pack_factor), so its name stays outside that list -- vLLM's own
    ``GPTQLinearMethod`` is in it."""

    def __init__(self, quant_config: GPTQLayerConfig):
        self.quant_config = quant_config

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs):
        cfg = self.quant_config
        bits = cfg.weight_bits
        k = input_size_per_partition
        n = sum(output_partition_sizes)
        gs = cfg.group_size if cfg.group_size != -1 else input_size
        if k % 32:
            raise ValueError(f"input size {k} must be a multiple of 32 for GPTQ packing")
        if (n * bits) % 32 or any((p * bits) % 32 for p in output_partition_sizes):
            raise ValueError(f"output sizes {output_partition_sizes} x {bits} bits must pack into int32")
        if gs % 32:
            raise ValueError(f"group_size {cfg.group_size} must be a multiple of 32 (or -1)")
        groups = (k + gs - 1) // gs
        offs = _shard_offsets(output_partition_sizes)
        loader = extra_weight_attrs.pop("weight_loader", None)

        def make_loader(out_dim: Optional[int], pack: int):
            def _load(param, loaded_weight: torch.Tensor, loaded_shard_id: Any = None):
                # g_idx (no output dim) is shared by every shard of a fused module
                if out_dim is None or len(output_partition_sizes) == 1 or loaded_shard_id is None:
                    param.data.copy_(loaded_weight)
                    return
                i = _shard_index(loaded_shard_id, len(output_partition_sizes))
                start, size = offs[i] // pack, output_partition_sizes[i] // pack
                param.data.narrow(out_dim, start, size).copy_(loaded_weight)

            return loader if loader is not None else _load

        qweight = torch.nn.Parameter(torch.empty(k * bits // 32, n, dtype=torch.int32), requires_grad=False)
        set_weight_attrs(qweight, {"input_dim": 0, "output_dim": 1, "packed_dim": 0,
                                   "pack_factor": cfg.pack_factor, "weight_loader": make_loader(1, 1),
                                   **extra_weight_attrs})
        g_idx = torch.nn.Parameter(torch.tensor([i // gs for i in range(k)], dtype=torch.int32),
                                   requires_grad=False)
        set_weight_attrs(g_idx, {"input_dim": 0, "ignore_warning": True,
                                 "weight_loader": make_loader(None, 1), **extra_weight_attrs})
        qzeros = torch.nn.Parameter(torch.empty(groups, n * bits // 32, dtype=torch.int32),
                                    requires_grad=False)
        set_weight_attrs(qzeros, {"input_dim": 0, "output_dim": 1, "packed_dim": 1,
                                  "pack_factor": cfg.pack_factor,
                                  "weight_loader": _zero_loader(loader, offs, output_partition_sizes, bits),
                                  **extra_weight_attrs})
        scales = torch.nn.Parameter(torch.empty(groups, n, dtype=torch.float16), requires_grad=False)
        set_weight_attrs(scales, {"input_dim": 0, "output_dim": 1,
                                  "weight_loader": make_loader(1, 1), **extra_weight_attrs})
        layer.register_parameter("qweight", qweight)
        layer.register_parameter("g_idx", g_idx)
        layer.register_parameter("qzeros", qzeros)
        layer.register_parameter("scales", scales)
        layer._oc_gptq = {"in": k, "out": n, "groups": groups, "gs": gs,
                          "parts": list(output_partition_sizes)}

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        cfg = self.quant_config
        dev = layer.qweight.device
        if dev.type != "cuda":
            raise RuntimeError("MixedGPTQLinearMethod needs the layer on a HIP device before "
                               "process_weights_after_loading")
        scales = layer.scales.data
        if scales.dtype != torch.float16:
            scales = scales.to(torch.float16)
        g_idx = layer.g_idx.data.to(torch.int32).contiguous()
        if not cfg.desc_act:
            gs = layer._oc_gptq["gs"]
            expected = torch.arange(g_idx.numel(), device=dev, dtype=torch.int32) // gs
            if torch.equal(g_idx, expected):
                g_idx = None
        layer._oc_prep = ops.gptq_prepare(layer.qweight.data.contiguous(), layer.qzeros.data.contiguous(),
                                          scales.contiguous(), g_idx, cfg.weight_bits,
                                          cfg.group_size, cfg.zero_format)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor,
              bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        prep = getattr(layer, "_oc_prep", None)
        if prep is None:
            raise RuntimeError("GPTQ layer used before process_weights_after_loading")
        if bias is not None and bias.dtype != x.dtype:
            bias = bias.to(x.dtype)
        return ops.gptq_gemm(x, prep, bias)


class MixedFusedGPTQLinearMethod(LinearMethodBase):
    """A fused module (qkv_proj, gate_up_proj) whose shards differ in bits or group size.

    The reference rejects such modules (vllm_plugins/gptq/vllm_plugin.py:310-317 via
    utils/module.py:153-177); with ``fused_mixed_bits`` enabled in the quantization config they
    are served as one ``apply()`` that runs every shard in one launch
    (``oc_gptq_gemm_grouped``).  Each checkpoint tensor of shard i (``q_proj.qweight`` etc.,
    AutoGPTQ layout at that shard's bits) is stored flat, back to back, in one parameter of the
    fused name, because the shards' packed shapes differ; ``g_idx`` is [n_shards, K].
    """

    def __init__(self, part_configs: List[GPTQLayerConfig]):
        self.part_configs = part_configs

    def create_weights(self, layer: torch.nn.Module, input_size_per_partition: int,
                       output_partition_sizes: List[int], input_size: int, output_size: int,
                       params_dtype: torch.dtype, **extra_weight_attrs):
        k = input_size_per_partition
        if len(output_partition_sizes) != len(self.part_configs):
            raise ValueError(f"{len(output_partition_sizes)} output partitions for "
                             f"{len(self.part_configs)} shard configs")
        if k % 32:
            raise ValueError(f"input size {k} must be a multiple of 32 for GPTQ packing")
        extra_weight_attrs.pop("weight_loader", None)
        shapes = {"qweight": [], "qzeros": [], "scales": []}
        groups = []
        for n, cfg in zip(output_partition_sizes, self.part_configs):
            b = cfg.weight_bits
            gs = cfg.group_size if cfg.group_size != -1 else input_size
            if (n * b) % 32 or gs % 32:
                raise ValueError(f"shard of {n} outputs at {b} bits / group {cfg.group_size} does not pack")
            g = (k + gs - 1) // gs
            groups.append(g)
            shapes["qweight"].append((k * b // 32, n))
            shapes["qzeros"].append((g, n * b // 32))
            shapes["scales"].append((g, n))
        n_shards = len(self.part_configs)

        def flat_param(name, dtype):
            offs, c = [], 0
            for shp in shapes[name]:
                offs.append(c)
                c += shp[0] * shp[1]
            prm = torch.nn.Parameter(torch.empty(c, dtype=dtype), requires_grad=False)

            def _load(param, loaded_weight: torch.Tensor, loaded_shard_id: Any = None):
                if loaded_shard_id is None:
                    raise ValueError(f"{name} of a fused module with per-shard bits needs a shard id")
                i = _shard_index(loaded_shard_id, n_shards)
                shp = shapes[name][i]
                if tuple(loaded_weight.shape) != shp:
                    raise ValueError(f"{name} shard {loaded_shard_id}: got {tuple(loaded_weight.shape)}, "
                                     f"expected {shp}")
                param.data[offs[i]:offs[i] + shp[0] * shp[1]].view(shp).copy_(loaded_weight)

            set_weight_attrs(prm, {"weight_loader": _load, "oc_shard_offsets": offs,
                                   "oc_shard_shapes": shapes[name], **extra_weight_attrs})
            return prm

        g_idx = torch.nn.Parameter(torch.stack([
            torch.tensor([i // (c.group_size if c.group_size != -1 else input_size) for i in range(k)],
                         dtype=torch.int32) for c in self.part_configs]), requires_grad=False)

        def _g_load(param, loaded_weight: torch.Tensor, loaded_shard_id: Any = None):
            if loaded_shard_id is None:
                param.data.copy_(loaded_weight.reshape(1, -1).expand_as(param.data))
                return
            param.data[_shard_index(loaded_shard_id, n_shards)].copy_(loaded_weight)

        set_weight_attrs(g_idx, {"weight_loader": _g_load, "ignore_warning": True, **extra_weight_attrs})
        layer.register_parameter("qweight", flat_param("qweight", torch.int32))
        layer.register_parameter("g_idx", g_idx)
        layer.register_parameter("qzeros", flat_param("qzeros", torch.int32))
        layer.register_parameter("scales", flat_param("scales", torch.float16))
        layer._oc_gptq = {"in": k, "out": sum(output_partition_sizes), "parts": list(output_partition_sizes),
                          "groups": groups}

    def shard_tensors(self, layer: torch.nn.Module, i: int):
        """(qweight, qzeros, scales, g_idx) views of shard i."""
        out = []
        for name in ("qweight", "qzeros", "scales"):
            p = getattr(layer, name)
            off, shp = p.oc_shard_offsets[i], p.oc_shard_shapes[i]
            out.append(p.data[off:off + shp[0] * shp[1]].view(shp))
        out.append(layer.g_idx.data[i])
        return out

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        dev = layer.qweight.device
        if dev.type != "cuda":
            raise RuntimeError("MixedFusedGPTQLinearMethod needs the layer on a HIP device before "
                               "process_weights_after_loading")
        preps = []
        for i, cfg in enumerate(self.part_configs):
            qw, qz, sc, g_idx = self.shard_tensors(layer, i)
            g_idx = g_idx.to(torch.int32).contiguous()
            if not cfg.desc_act:
                gs = cfg.group_size if cfg.group_size != -1 else layer._oc_gptq["in"]
                expected = torch.arange(g_idx.numel(), device=dev, dtype=torch.int32) // gs
                if torch.equal(g_idx, expected):
                    g_idx = None
            preps.append(ops.gptq_prepare(qw.contiguous(), qz.contiguous(), sc.to(torch.float16).contiguous(),
                                          g_idx, cfg.weight_bits, cfg.group_size, cfg.zero_format))
        layer._oc_preps = preps

    def apply(self, layer: torch.nn.Module, x: torch.Tensor,
              bias: Optional[torch.Tensor] = None) -> torch.Tensor:
        preps = getattr(layer, "_oc_preps", None)
        if preps is None:
            raise RuntimeError("GPTQ layer used before process_weights_after_loading")
        biases = None
        if bias is not None:
            b = bias.to(x.dtype) if bias.dtype != x.dtype else bias
            biases, off = [], 0
            for p in preps:
                biases.append(b[off:off + p.out_features])
                off += p.out_features
        return ops.gptq_gemm_grouped(x, preps, biases)


def _zero_loader(loader, offs, parts, bits):
    """qzeros are packed along N: shard i occupies columns offs[i]*b/32 ..."""
    if loader is not None:
        return loader

    def _load(param, loaded_weight: torch.Tensor, loaded_shard_id: Any = None):
        if len(parts) == 1 or loaded_shard_id is None:
            param.data.copy_(loaded_weight)
            return
        i = _shard_index(loaded_shard_id, len(parts))
        start, size = offs[i] * bits // 32, parts[i] * bits // 32
        param.data.narrow(1, start, size).copy_(loaded_weight)

    return _load


class GPTQMoEMethod(QuantizeMethodBase):
    """FusedMoE method over GPTQ experts.

    Replaces the vLLM WNA16 method that ``MixedGPTQConfig._get_moe_quant_method`` builds
    (vllm_plugins/gptq/vllm_plugin.py:241-283) and its gpt-oss variant with expert bias and the
    swigluoai activation (gptoss_wna16_moe.py:55-175).  The experts' AutoGPTQ tensors are
    registered expert-stacked, gate and up side by side (gate columns first):
    ``w13_qweight`` [E, H·b/32, 2I], ``w13_qzeros`` [E, G, 2I·b/32], ``w13_scales`` [E, G, 2I],
    ``w2_*`` likewise for down (I -> H), and with ``layer.has_bias`` ``w13_bias`` [E, 2I],
    ``w2_bias`` [E, H].  The loader takes FusedMoE's ``(param, loaded, weight_name, shard_id,
    expert_id)`` with shard_id ``w1`` (gate), ``w3`` (up) or ``w2`` (down).  After loading the
    experts are repacked once (``moe.prepare_experts_merged``) and the checkpoint tensors freed;
    ``apply`` runs ``oc_moe_gptq_forward``.  With ``desc_act`` the experts' act-order g_idx are
    registered as ``w13_g_idx`` [E, H] (gate and up load into one row per expert and must agree:
    the merged gate|up layer has one k order) and ``w2_g_idx`` [E, I].  ``apply_router_weight_on_input``
    (top-1) scales the input rows by the router weight before the experts.
    """

    _ACT = {"silu": "silu", "swigluoai": "gpt_oss", "gelu": "gelu_pytorch_tanh"}

    def __init__(self, quant_config: GPTQLayerConfig):
        self.quant_config = quant_config

    def create_weights(self, layer: torch.nn.Module, num_experts: int, hidden_size: int,
                       intermediate_size_per_partition: int, params_dtype: torch.dtype, **extra_weight_attrs):
        cfg = self.quant_config
        bits, E, H, I = cfg.weight_bits, num_experts, hidden_size, intermediate_size_per_partition
        if H % 32 or I % 32:
            raise ValueError(f"hidden {H} and intermediate {I} sizes must be multiples of 32")
        gs13 = cfg.group_size if cfg.group_size != -1 else H
        gs2 = cfg.group_size if cfg.group_size != -1 else I
        if gs13 % 32 or gs2 % 32:
            raise ValueError(f"group_size {cfg.group_size} must be a multiple of 32 (or -1)")
        g13, g2 = (H + gs13 - 1) // gs13, (I + gs2 - 1) // gs2
        extra_weight_attrs.pop("weight_loader", None)
        shapes = {
            "w13_qweight": ((E, H * bits // 32, 2 * I), torch.int32),
            "w13_qzeros": ((E, g13, 2 * I * bits // 32), torch.int32),
            "w13_scales": ((E, g13, 2 * I), torch.float16),
            "w2_qweight": ((E, I * bits // 32, H), torch.int32),
            "w2_qzeros": ((E, g2, H * bits // 32), torch.int32),
            "w2_scales": ((E, g2, H), torch.float16),
        }
        if getattr(layer, "has_bias", False):
            shapes["w13_bias"] = ((E, 2 * I), params_dtype)
            shapes["w2_bias"] = ((E, H), params_dtype)
        if cfg.desc_act:
            shapes["w13_g_idx"] = ((E, H), torch.int32)
            shapes["w2_g_idx"] = ((E, I), torch.int32)
        for name, (shape, dtype) in shapes.items():
            param = torch.nn.Parameter(torch.zeros(shape, dtype=dtype), requires_grad=False)
            layer.register_parameter(name, param)
            set_weight_attrs(param, {"weight_loader": self._load, **extra_weight_attrs})
        layer._oc_moe = {"E": E, "H": H, "I": I}

    @staticmethod
    def _load(param, loaded_weight: torch.Tensor, weight_name: str, shard_id: str, expert_id: int,
              return_success: bool = False):
        """Place one expert's gate (w1) / up (w3) half of a w13 tensor, or its down (w2) tensor; a
        g_idx row (act-order) is shared by w1 and w3, which must agree."""
        dst = param.data[expert_id]
        if "g_idx" in weight_name:
            if shard_id not in ("w1", "w3", "w2") or (shard_id == "w2") != ("w2" in weight_name):
                raise ValueError(f"{weight_name}: unexpected shard_id {shard_id!r}")
            if tuple(loaded_weight.shape) != tuple(dst.shape):
                raise ValueError(f"{weight_name} expert {expert_id} shard {shard_id}: checkpoint shape "
                                 f"{tuple(loaded_weight.shape)} != {tuple(dst.shape)}")
            g = loaded_weight.to(device=dst.device, dtype=dst.dtype)
            seen = getattr(param, "_oc_g_idx_seen", None)
            if seen is None:
                seen = {}
                param._oc_g_idx_seen = seen
            other = seen.get((expert_id, "w3" if shard_id == "w1" else "w1")) if shard_id != "w2" else None
            if other is not None and not torch.equal(other, g):
                raise ValueError(f"expert {expert_id}: act-order gate_proj and up_proj g_idx differ; the merged "
                                 "gate|up layer needs one k order")
            if shard_id != "w2":
                seen[(expert_id, shard_id)] = g
            dst.copy_(g)
            return True if return_success else None
        if "w13" in weight_name:
            if shard_id not in ("w1", "w3"):
                raise ValueError(f"{weight_name}: shard_id must be w1 or w3, got {shard_id!r}")
            half = dst.shape[-1] // 2
            dst = dst.narrow(dst.dim() - 1, 0 if shard_id == "w1" else half, half)
        elif shard_id != "w2":
            raise ValueError(f"{weight_name}: shard_id must be w2, got {shard_id!r}")
        if tuple(loaded_weight.shape) != tuple(dst.shape):
            raise ValueError(f"{weight_name} expert {expert_id} shard {shard_id}: checkpoint shape "
                             f"{tuple(loaded_weight.shape)} != {tuple(dst.shape)}")
        dst.copy_(loaded_weight.to(device=dst.device, dtype=dst.dtype))
        return True if return_success else None

    def process_weights_after_loading(self, layer: torch.nn.Module) -> None:
        from . import moe

        cfg = self.quant_config
        if layer.w13_qweight.device.type != "cuda":
            raise RuntimeError("GPTQMoEMethod needs the layer on a HIP device before process_weights_after_loading")
        b13 = getattr(layer, "w13_bias", None)
        b2 = getattr(layer, "w2_bias", None)
        g13 = getattr(layer, "w13_g_idx", None)
        g2 = getattr(layer, "w2_g_idx", None)
        layer._oc_experts = moe.prepare_experts_merged(
            layer.w13_qweight.data, layer.w13_qzeros.data, layer.w13_scales.data, layer.w2_qweight.data,
            layer.w2_qzeros.data, layer.w2_scales.data, cfg.weight_bits, cfg.group_size, cfg.zero_format,
            None if b13 is None else b13.data, None if b2 is None else b2.data,
            None if g13 is None else g13.data, None if g2 is None else g2.data)
        if g13 is not None:
            g13._oc_g_idx_seen = None
        for name in ("w13_qweight", "w13_qzeros", "w13_scales", "w2_qweight", "w2_qzeros", "w2_scales"):
            getattr(layer, name).data = torch.empty(0, dtype=getattr(layer, name).dtype,
                                                    device=layer.w13_qweight.device)

    def apply(self, layer: torch.nn.Module, x: torch.Tensor, topk_weights: torch.Tensor,
              topk_ids: torch.Tensor, shared_experts_input: Optional[torch.Tensor] = None) -> torch.Tensor:
        from . import moe

        ex = getattr(layer, "_oc_experts", None)
        if ex is None:
            raise RuntimeError("GPTQ MoE layer used before process_weights_after_loading")
        if getattr(layer, "expert_map", None) is not None:
            raise NotImplementedError("expert parallelism (expert_map) is not supported")
        act = str(getattr(layer, "activation", "silu")).lower().rsplit(".", 1)[-1]
        if act not in self._ACT:
            raise NotImplementedError(f"MoE activation {act!r}; supported: {sorted(self._ACT)}")
        return moe.moe_forward(x, topk_ids, topk_weights, ex, self._ACT[act],
                               router_weight_on_input=bool(getattr(layer, "apply_router_weight_on_input", False)))


@register_quantization_config("mixed_gptq")
class MixedGPTQConfig(QuantizationConfig):
    """``quant_method: mixed_gptq`` (vllm_plugins/gptq/vllm_plugin.py:83-365)."""

    def __init__(self, quantization_bits, group_size=-1, desc_act=False, sym=False,
                 lm_head_quantized=False, checkpoint_format="gptq_v2",
                 rotation_metadata: Optional[RotationMetadata] = None, fused_mixed_bits: bool = False):
        super().__init__()
        self.quantization_bits = quantization_bits  # one {module name: entry} dict per decoder layer
        self.group_size, self.desc_act, self.sym = group_size, desc_act, sym
        self.lm_head_quantized = lm_head_quantized
        self.checkpoint_format = checkpoint_format
        self.rotation_metadata = rotation_metadata or RotationMetadata()
        # This build's extension, off unless the config asks for it: serve fused modules whose
        # shards differ in bits or group size instead of raising ValueError.
        self.fused_mixed_bits = bool(fused_mixed_bits)
        entries = [e for per_layer in quantization_bits for e in per_layer.values()]
        logger.info("mixed_gptq over %d decoder layers: bit widths %s, methods %s", len(quantization_bits),
                    sorted({e.get("bits", 0) for e in entries}), sorted({e.get("method", "gptq") for e in entries}))

    def __repr__(self):
        return (f"MixedGPTQConfig(num_layers={len(self.quantization_bits)}, group_size={self.group_size}, "
                f"desc_act={self.desc_act}, checkpoint_format={self.checkpoint_format!r})")

    @classmethod
    def get_name(cls) -> str:
        return "mixed_gptq"

    @classmethod
    def get_supported_act_dtypes(cls) -> List[torch.dtype]:
        return [torch.half, torch.bfloat16]

    @classmethod
    def get_min_capability(cls) -> int:
        return 60

    @staticmethod
    def get_config_filenames() -> List[str]:
        return ["quantize_config.json"]

    @classmethod
    def from_config(cls, config: Dict[str, Any]) -> "MixedGPTQConfig":
        quantization_bits = config.get("quantization_bits", [])
        if not quantization_bits and "layer_bits" in config:
            quantization_bits = [{"_all": {"bits": b, "method": "gptq"}} for b in config["layer_bits"]]
        return cls(quantization_bits=quantization_bits,
                   group_size=config.get("group_size", -1),
                   desc_act=config.get("desc_act", False),
                   sym=config.get("sym", False),
                   lm_head_quantized=config.get("lm_head", False),
                   checkpoint_format=config.get("checkpoint_format", "gptq_v2"),
                   rotation_metadata=RotationMetadata.from_quant_config(config),
                   fused_mixed_bits=config.get("fused_mixed_bits", False))

    def maybe_update_config(self, model_name, hf_config=None, revision=None):
        """No-op: per-module dispatch comes from ``quantization_bits`` (vllm_plugin.py:213-218)."""

    def _resolve_group_size(self, mod_cfg: Optional[Dict]) -> int:
        """Group size of one module entry: the entry's own ``group_size``, else the one in its
        ``params`` dict, else the config-wide value (vllm_plugin.py:165-173)."""
        if mod_cfg is None:
            return self.group_size
        nested = mod_cfg.get("params")
        for candidate in (mod_cfg.get("group_size"), nested.get("group_size") if isinstance(nested, dict) else None):
            if candidate is not None:
                return candidate
        return self.group_size

    resolve_group_size = _resolve_group_size

    def _mixed_fused_method(self, layer_idx: int, suffix: str, prefix: str):
        """MixedFusedGPTQLinearMethod when enabled and every shard is a GPTQ entry, else None."""
        if not self.fused_mixed_bits:
            return None
        cfgs = constituent_configs(self.quantization_bits, layer_idx, suffix)
        if not cfgs or any(c is None for c in cfgs):
            return None
        parts = []
        for c in cfgs:
            bits = int(c.get("bits", 0))
            if c.get("method", "gptq") != "gptq" or bits not in SUPPORTED_BITS:
                return None
            parts.append(GPTQLayerConfig(bits, self.resolve_group_size(c), self.desc_act, bool(self.sym),
                                         self.checkpoint_format))
        return maybe_wrap_rotation_method(MixedFusedGPTQLinearMethod(parts), prefix=prefix,
                                          metadata=self.rotation_metadata)

    def _unquantized(self, prefix: str):
        return maybe_wrap_rotation_method(UnquantizedLinearMethod(), prefix=prefix,
                                          metadata=self.rotation_metadata)

    def _lookup_moe_expert_config(self, layer_idx: int) -> Optional[Dict[str, Any]]:
        """The entry that configures a MoE layer's experts (all experts share bits and group size,
        vllm_plugin.py:220-239): among the layer's ``experts.<i>.`` entries, the first gate_proj,
        else the first up_proj, else the first down_proj, else the first of any kind."""
        if not 0 <= layer_idx < len(self.quantization_bits):
            return None
        preference = (".gate_proj", ".up_proj", ".down_proj")

        def rank(name: str) -> int:
            return next((i for i, suffix in enumerate(preference) if name.endswith(suffix)), len(preference))

        experts = [(rank(n), i, c) for i, (n, c) in enumerate(self.quantization_bits[layer_idx].items())
                   if _MOE_EXPERT_CFG_RE.search(n)]
        return min(experts, key=lambda t: t[:2])[2] if experts else None

    def _get_moe_quant_method(self, layer: torch.nn.Module, prefix: str):
        """GPTQMoEMethod for a FusedMoE layer with per-expert GPTQ entries, else None (unquantized
        experts), as vllm_plugin.py:241-283 decides."""
        layer_idx, _ = parse_layer_and_module(prefix)
        if layer_idx is None:
            return None
        mod_cfg = self._lookup_moe_expert_config(layer_idx)
        if mod_cfg is None:
            return None
        bits = int(mod_cfg.get("bits", 0))
        if bits == 0 or mod_cfg.get("method", "gptq") != "gptq":
            return None
        return GPTQMoEMethod(GPTQLayerConfig(bits, self.resolve_group_size(mod_cfg), self.desc_act,
                                             bool(self.sym), self.checkpoint_format))

    def get_quant_method(self, layer: torch.nn.Module, prefix: str):
        if FusedMoE is not None and isinstance(layer, FusedMoE):
            return self._get_moe_quant_method(layer, prefix)
        if not isinstance(layer, LinearBase):
            return None
        layer_idx, suffix = parse_layer_and_module(prefix)
        if layer_idx is None:
            return self._unquantized(prefix)
        mod_cfg = lookup_module_config(self.quantization_bits, layer_idx, suffix)
        if mod_cfg is None:
            return self._unquantized(prefix)
        if not validate_quant_config_within_shard(self.quantization_bits, layer_idx, suffix):
            mixed = self._mixed_fused_method(layer_idx, suffix, prefix)
            if mixed is not None:
                return mixed
            raise ValueError(f"Detected some but not all shards of {prefix} are quantized. "
                             "All shards of fused layers to have the same precision.")
        bits = mod_cfg.get("bits", 0)
        method = mod_cfg.get("method", "gptq")
        if bits == 0:
            return self._unquantized(prefix)
        if method == "gptq" and int(bits) in SUPPORTED_BITS:
            cfg = GPTQLayerConfig(int(bits), self.resolve_group_size(mod_cfg), self.desc_act,
                                  bool(self.sym), self.checkpoint_format)
            return maybe_wrap_rotation_method(MixedGPTQLinearMethod(cfg), prefix=prefix,
                                              metadata=self.rotation_metadata)
        logger.warning("mixed_gptq: unsupported method=%s bits=%s at %s, falling back to unquantized",
                       method, bits, prefix)
        return self._unquantized(prefix)


def register_vllm_plugin():
    """vLLM ``general_plugins`` entry point (vllm_plugin.py:368-373)."""
    register_quantization_config(MixedGPTQConfig)
