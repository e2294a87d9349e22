"""Rotated (SpinQuant/OstQuant-preprocessed) checkpoints: metadata and the online Hadamard.

Mirrors vllm_plugins/utils/rotation.py:
- ``RotationMetadata`` (:75-97) and the target predicate of
  onecomp/pre_process/rotation_utils.py:125-136;
- ``RotatedLinearMethod`` (:146-228): wraps a layer's linear method and
  transforms the ``mlp.down_proj`` input online, y = (H_K (x) H_L) x / sqrt(n),
  through a forward pre-hook installed at create_weights /
  process_weights_after_loading, as the reference does for tp = 1.  The
  transform is ``ops.hadamard`` (one HIP launch: the length-L transforms in
  fp32, then the K x K mix on MFMA with fp32 accumulation; up to 16 rows as
  products over L / 16 workgroups per row, from 32 rows one workgroup per
  row), rounded as the metadata's ``fp32_had`` asks: True keeps fp32 and
  rounds once; False (the default) rounds every butterfly stage (the
  reference's pure-PyTorch transform; once with FAST_HADAMARD_TRANSFORM),
  the 1/sqrt(n) division and the H_K product;
- ``maybe_wrap_rotation_method`` (:242-261).
Tensor parallelism > 1 needs an all-gather of the input first (:179-195);
this one-GPU build raises for it.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional

from .vllm_compat import LinearMethodBase, WEIGHT_LOADER_V2_SUPPORTED, register_weight_loader_v2_supported_method


def is_online_hadamard_target(name: str) -> bool:
    """Dense ``mlp.down_proj`` layers receive the online Hadamard."""
    return name == "mlp.down_proj" or name.endswith(".mlp.down_proj")


@dataclass(frozen=True)
class RotationMetadata:
    rotated: bool = False
    fp32_had: bool = False

    @classmethod
    def from_quant_config(cls, config: Optional[Dict[str, Any]]) -> "RotationMetadata":
        if not isinstance(config, dict):
            return cls()
        return cls(rotated=bool(config.get("rotated", False)),
                   fp32_had=bool(config.get("fp32_had", False)))

    def requires_hadamard(self, prefix: str) -> bool:
        return self.rotated and is_online_hadamard_target(prefix)


# The reference's transform op is the fast_hadamard_transform package when it is installed,
# else its pure-PyTorch butterflies (hadamard_utils.py:17-68); its dependencies do not include the
# package, so fp32_had=False follows the butterflies' per-stage rounding unless this is set.
FAST_HADAMARD_TRANSFORM = False


def apply_online_hadamard(x, *, fp32_had: bool = False, cache_owner: Any = None):
    """Online Hadamard of the last axis (rotation.py:100-112); the block order is cached on the owner."""
    from . import ops

    if cache_owner is not None:
        cached = getattr(cache_owner, "_onecomp_hadamard_cache", None)
        if cached is None or cached[0] != x.shape[-1]:
            setattr(cache_owner, "_onecomp_hadamard_cache", (x.shape[-1], ops.hadamard_order(x.shape[-1])))
    rounding = "fp32" if fp32_had else ("once" if FAST_HADAMARD_TRANSFORM else "stages")
    return ops.hadamard(x, rounding=rounding)


def make_hadamard_forward_pre_hook(*, fp32_had: bool):
    """Layer pre-hook that transforms the first positional input (rotation.py:115-125)."""

    def hook(layer, inputs):
        if not inputs:
            return inputs
        return (apply_online_hadamard(inputs[0], fp32_had=fp32_had, cache_owner=layer), *inputs[1:])

    return hook


class RotatedLinearMethod(LinearMethodBase):
    """Linear-method wrapper that transforms the layer input online (rotation.py:146-228).

    Not on vLLM's v2 weight-loader list: it wraps base methods whose params take the v1 loader
    (vLLM picks the loader by the wrapper's class name).  :class:`RotatedLinearMethodV2` is the
    listed twin for v2-native bases."""

    def __init__(self, base_method, *, fp32_had: bool):
        self.base_method = base_method
        self.fp32_had = fp32_had

    def _check_tp(self, layer) -> None:
        tp_size = getattr(layer, "tp_size", 1) or 1
        if getattr(layer, "input_is_parallel", False) and tp_size > 1:
            raise NotImplementedError("tensor-parallel rotated down_proj needs an all-gather before the "
                                      "Hadamard; this build runs one GPU")

    def _ensure_hadamard_pre_hook(self, layer) -> None:
        self._check_tp(layer)
        if getattr(layer, "_onecomp_hadamard_prehook_installed", False):
            return
        handle = layer.register_forward_pre_hook(make_hadamard_forward_pre_hook(fp32_had=self.fp32_had))
        setattr(layer, "_onecomp_hadamard_prehook_installed", True)
        setattr(layer, "_onecomp_hadamard_prehook_handle", handle)

    def create_weights(self, layer, *weight_args, **extra_weight_attrs):
        self._ensure_hadamard_pre_hook(layer)
        return self.base_method.create_weights(layer, *weight_args, **extra_weight_attrs)

    def process_weights_after_loading(self, layer) -> None:
        self._ensure_hadamard_pre_hook(layer)
        process = getattr(self.base_method, "process_weights_after_loading", None)
        if process is not None:
            process(layer)

    def apply(self, layer, x, bias=None, *args, **kwargs):
        return self.base_method.apply(layer, x, bias, *args, **kwargs)

    def __getattr__(self, name):  # expose the wrapped method's extras (e.g. quant_config)
        return getattr(self.base_method, name)


@register_weight_loader_v2_supported_method
class RotatedLinearMethodV2(RotatedLinearMethod):
    """The wrapper for base methods on vLLM's v2 weight-loader list (rotation.py:232-239)."""


def _takes_v2_loader(method) -> bool:
    """Whether vLLM would give ``method``'s layer the v2 weight loader (by class name); with no
    inspectable list, assume v2, as the reference does (rotation.py:126-144)."""
    if WEIGHT_LOADER_V2_SUPPORTED is None:
        return True
    return type(method).__name__ in WEIGHT_LOADER_V2_SUPPORTED


def maybe_wrap_rotation_method(method, *, prefix: str, metadata: RotationMetadata):
    """``method`` unchanged, or wrapped with the online Hadamard for rotated down_proj layers; the
    wrapper keeps the base method's v1/v2 loader choice (rotation.py:242-261)."""
    if not metadata.requires_hadamard(prefix):
        return method
    cls = RotatedLinearMethodV2 if _takes_v2_loader(method) else RotatedLinearMethod
    return cls(method, fp32_had=metadata.fp32_had)
