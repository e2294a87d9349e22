"""Per-module config lookup for ``quantization_bits`` (host logic, no GPU).

Same rules as vllm_plugins/utils/module.py:
- the layer index is the number after ``.layers.`` in the vLLM prefix, and
  vision/audio encoder prefixes are never quantized (:51-59);
- a module's entry is the first key its suffix starts with, then the entry of
  a constituent of a fused module (qkv_proj -> q/k/v_proj, gate_up_proj ->
  gate/up_proj), then the layer's ``_all`` entry (:74-89);
- a fused module is servable only if every constituent has an entry and all
  entries are equal (:139-177);
- vLLM's ``attn.*`` suffixes alias the checkpoint's ``self_attn.*`` (:40-48).
"""

from __future__ import annotations

import re
from typing import Dict, List, Optional, Tuple

LAYER_RE = re.compile(r"\.layers\.(\d+)\.")
NON_TEXT_PREFIXES = ("vision_tower", "vision_model", "multi_modal_projector", "audio")
FUSED_TO_CONSTITUENTS = {
    "qkv_proj": ["q_proj", "k_proj", "v_proj"],
    "gate_up_proj": ["gate_proj", "up_proj"],
}
SUFFIX_ALIASES = (("attn.", "self_attn."),)


def normalize_module_suffix(suffix: str) -> str:
    for src, dst in SUFFIX_ALIASES:
        if suffix.startswith(src):
            return dst + suffix[len(src):]
    return suffix


def parse_layer_and_module(prefix: str) -> Tuple[Optional[int], Optional[str]]:
    """(layer index, module suffix) of a vLLM prefix, or (None, None)."""
    if any(p in prefix for p in NON_TEXT_PREFIXES):
        return None, None
    m = LAYER_RE.search(prefix)
    if m is None:
        return None, None
    return int(m.group(1)), prefix[m.end():]


def _fused_entry(layer_cfg: Dict, suffix: str) -> Optional[Dict]:
    for fused, parts in FUSED_TO_CONSTITUENTS.items():
        if fused not in suffix:
            continue
        for part in parts:
            cand = suffix.replace(fused, part)
            if cand in layer_cfg:
                return layer_cfg[cand]
        return None
    return None


def lookup_module_config(quantization_bits: List[Dict], layer_idx: int, suffix: str) -> Optional[Dict]:
    if layer_idx >= len(quantization_bits):
        return None
    layer_cfg = quantization_bits[layer_idx]
    suffix = normalize_module_suffix(suffix)
    for name, cfg in layer_cfg.items():
        if suffix.startswith(name):
            return cfg
    fused = _fused_entry(layer_cfg, suffix)
    if fused is not None:
        return fused
    return layer_cfg.get("_all")


def constituent_configs(quantization_bits: List[Dict], layer_idx: int, suffix: str) -> Optional[List[Dict]]:
    """Entries of a fused module's constituents in order, or None if not fused."""
    if layer_idx >= len(quantization_bits):
        return None
    layer_cfg = quantization_bits[layer_idx]
    suffix = normalize_module_suffix(suffix)
    for fused, parts in FUSED_TO_CONSTITUENTS.items():
        if fused in suffix:
            return [layer_cfg.get(suffix.replace(fused, p)) for p in parts]
    return None


def validate_quant_config_within_shard(quantization_bits: List[Dict], layer_idx: int, suffix: str) -> bool:
    """True unless a fused module has a missing or differing constituent entry."""
    if layer_idx >= len(quantization_bits):
        return False
    cfgs = constituent_configs(quantization_bits, layer_idx, suffix)
    if cfgs is None:
        return True
    if any(c is None for c in cfgs):
        return False
    return all(c == cfgs[0] for c in cfgs)
