"""Seeded synthetic checkpoints and activations for the benchmark configs.

Generated on the CPU with ``torch.Generator(device="cpu").manual_seed(seed)``
so every consumer (GPU path, CPU baseline, tests) sees identical bytes, then
copied to the requested device.  Uniform codes are produced directly as
uniform random packed words: every bit of a packed word is an independent fair
bit, so each b-bit code (including the 3-bit codes that straddle words) is
uniform on [0, 2^b - 1], exactly as the configs ask.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import torch


@dataclass
class GPTQCase:
    name: str
    in_features: int
    out_features: int
    bits: int
    group_size: int
    act_order: bool
    qweight: torch.Tensor  # int32 [K*b/32, N]
    qzeros: torch.Tensor   # int32 [G, N*b/32] (stored v1 fields)
    scales: torch.Tensor   # fp16 [G, N]
    g_idx: Optional[torch.Tensor]  # int32 [K] or None

    def weight_bytes(self) -> int:
        n = self.qweight.numel() * 4 + self.qzeros.numel() * 4 + self.scales.numel() * 2
        if self.g_idx is not None:
            n += self.g_idx.numel() * 4
        return n

    def to(self, dev):
        return GPTQCase(self.name, self.in_features, self.out_features, self.bits, self.group_size,
                        self.act_order, self.qweight.to(dev), self.qzeros.to(dev),
                        self.scales.to(dev), None if self.g_idx is None else self.g_idx.to(dev))


def _words(gen, shape):
    return torch.randint(-(2**31), 2**31, shape, generator=gen, dtype=torch.int64).to(torch.int32)


def gptq_case(name, k, n, bits, group_size=128, act_order=False, seed=0) -> GPTQCase:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    gs = k if group_size <= 0 else group_size
    g = (k + gs - 1) // gs
    qweight = _words(gen, (k * bits // 32, n))
    qzeros = _words(gen, (g, n * bits // 32))
    scales = (torch.randn((g, n), generator=gen).abs() * 0.02 + 1e-3).to(torch.float16)
    g_idx = None
    if act_order:
        perm = torch.randperm(k, generator=gen)
        g_idx = (torch.argsort(perm) // gs).to(torch.int32)
    return GPTQCase(name, k, n, bits, group_size, act_order, qweight, qzeros, scales, g_idx)


def activations(m, k, dtype=torch.float16, seed=1) -> torch.Tensor:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    return torch.randn((m, k), generator=gen).to(dtype)


# BASELINE configs (shapes and bit widths) -------------------------------------------------
CONFIG0 = [("linear", 4096, 4096, 4)]
CONFIG1 = [  # Llama-3-8B decoder layer, Mixed-GPTQ per projection
    ("q_proj", 4096, 4096, 4),
    ("k_proj", 4096, 1024, 8),
    ("v_proj", 4096, 1024, 8),
    ("o_proj", 4096, 4096, 4),
    ("gate_proj", 4096, 14336, 3),
    ("up_proj", 4096, 14336, 3),
    ("down_proj", 14336, 4096, 2),
]
CONFIG2 = [  # Qwen3-8B MLP, 3-bit act-order
    ("gate_proj", 4096, 12288, 3),
    ("up_proj", 4096, 12288, 3),
    ("down_proj", 12288, 4096, 3),
]
CONFIG4 = [  # Qwen3-14B prefill, 4-bit, bf16 activations
    ("qkv_proj", 5120, 7168, 4),
    ("o_proj", 5120, 5120, 4),
    ("gate_up_proj", 5120, 34816, 4),
    ("down_proj", 17408, 5120, 4),
]


def fuse_cases(cases, name: str) -> GPTQCase:
    """Concatenate same-K, same-bits, no-act-order projections along N.

    This is how vLLM stores a merged layer (QKVParallelLinear /
    MergedColumnParallelLinear): one qweight/qzeros/scales whose output
    columns are the shards side by side, served by one apply() call.
    """
    c0 = cases[0]
    for c in cases:
        if (c.in_features, c.bits, c.group_size, c.act_order) != (c0.in_features, c0.bits, c0.group_size, False):
            raise ValueError(f"cannot fuse {c.name} with {c0.name}")
        if (c.out_features * c.bits) % 32:
            raise ValueError(f"{c.name}: N * bits must be a multiple of 32 to concatenate packed zeros")
    return GPTQCase(name, c0.in_features, sum(c.out_features for c in cases), c0.bits, c0.group_size, False,
                    torch.cat([c.qweight for c in cases], dim=1), torch.cat([c.qzeros for c in cases], dim=1),
                    torch.cat([c.scales for c in cases], dim=1), None)


# Projections that read the same input and share bits / group size run as one
# merged layer, as vLLM builds them (q stays alone when its bits differ).
LAYER_GROUPS = {1: [("q_proj",), ("k_proj", "v_proj"), ("o_proj",), ("gate_proj", "up_proj"), ("down_proj",)]}


def layer_cases(cfg: int, seed: int = 0):
    """The apply() calls of one decoder layer: config cases, merged per LAYER_GROUPS."""
    cases = config_cases(cfg, seed)
    groups = LAYER_GROUPS.get(cfg)
    if groups is None:
        return cases
    by_name = {c.name: c for c in cases}
    out = []
    for g in groups:
        out.append(by_name[g[0]] if len(g) == 1 else fuse_cases([by_name[n] for n in g], "_".join(
            [g[0].replace("_proj", "")] + [n.replace("_proj", "") for n in g[1:]]) + "_proj"))
    return out


def layer_calls(cfg: int, seed: int = 0):
    """The apply() calls of one decoder layer as a fused-module plugin issues them: a list of
    calls, each a list of parts.  Same-bits shards are merged into one part (vLLM's merged
    layers); a call with several parts is a fused module whose shards differ in bits
    (q@4b with k, v@8b as one qkv_proj, served by oc_gptq_gemm_grouped)."""
    if cfg != 1:
        return [[c] for c in layer_cases(cfg, seed)]
    by_name = {c.name: c for c in config_cases(cfg, seed)}
    kv = fuse_cases([by_name["k_proj"], by_name["v_proj"]], "k_v_proj")
    gu = fuse_cases([by_name["gate_proj"], by_name["up_proj"]], "gate_up_proj")
    return [[by_name["q_proj"], kv], [by_name["o_proj"]], [gu], [by_name["down_proj"]]]


def config_cases(cfg: int, seed: int = 0):
    spec = {0: CONFIG0, 1: CONFIG1, 2: CONFIG2, 4: CONFIG4}[cfg]
    act = cfg == 2
    return [gptq_case(name, k, n, b, 128, act, seed + i) for i, (name, k, n, b) in enumerate(spec)]


# DBF / MDBF (config 3) ---------------------------------------------------------------------
CONFIG3 = [("up_proj", 4096, 14336), ("down_proj", 14336, 4096)]


def dbf_rank(bits: float, k: int, n: int) -> int:
    """DBF rank as the reference computes it (int() truncation, capped at min(K, N))."""
    return min(min(k, n), int(bits * k * n / (k + n)))


def _signs(gen, rows: int, cols: int) -> torch.Tensor:
    """rows x cols +-1 factor bit-packed MSB-first, flat (uniform random bits)."""
    nbytes = (rows * cols + 7) // 8
    return torch.randint(0, 256, (nbytes,), generator=gen, dtype=torch.int64).to(torch.uint8)


def _vec(gen, n: int) -> torch.Tensor:
    return (torch.randn(n, generator=gen).abs() * 0.05 + 1e-3).to(torch.float16)


@dataclass
class DBFCase:
    """One DBF path W = diag(s4) S1 diag(s2) S2 diag(s0) in the checkpoint layout."""

    name: str
    in_features: int
    out_features: int
    mid: int
    s0: torch.Tensor   # fp16 [K]
    bp1: torch.Tensor  # uint8, S2 (r x K)
    s2: torch.Tensor   # fp16 [r]
    bp3: torch.Tensor  # uint8, S1 (N x r)
    s4: torch.Tensor   # fp16 [N]

    def weight_bytes(self) -> int:
        return (self.bp1.numel() + self.bp3.numel() +
                2 * (self.in_features + self.mid + self.out_features))

    def to(self, dev):
        return DBFCase(self.name, self.in_features, self.out_features, self.mid, self.s0.to(dev),
                       self.bp1.to(dev), self.s2.to(dev), self.bp3.to(dev), self.s4.to(dev))


def dbf_case(name: str, k: int, n: int, bits: float = 1.0, seed: int = 0) -> DBFCase:
    gen = torch.Generator(device="cpu").manual_seed(seed)
    r = dbf_rank(bits, k, n)
    return DBFCase(name, k, n, r, _vec(gen, k), _signs(gen, r, k), _vec(gen, r), _signs(gen, n, r),
                   _vec(gen, n))
