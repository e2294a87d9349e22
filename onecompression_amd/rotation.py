"""Rotation metadata of rotated (SpinQuant/OstQuant-preprocessed) checkpoints.

Mirrors vllm_plugins/utils/rotation.py:75-97 (``RotationMetadata``) and the
target predicate of onecomp/pre_process/rotation_utils.py:125-136.  A rotated
checkpoint needs an online Hadamard transform of the ``mlp.down_proj`` input
(vllm_plugins/utils/rotation.py:146-261).  That transform is not built here
yet, so asking for it raises instead of silently computing wrong outputs.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Any, Dict, Optional


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


def maybe_wrap_rotation_method(method, *, prefix: str, metadata: RotationMetadata):
    """Return ``method`` unchanged, or raise for layers that need the online Hadamard."""
    if not metadata.requires_hadamard(prefix):
        return method
    raise NotImplementedError(
        f"{prefix}: rotated checkpoints need the online Hadamard transform of the down_proj "
        "input, which onecomp-amd does not implement yet")
