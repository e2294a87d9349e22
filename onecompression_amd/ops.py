"""Torch-tensor front end of the C ABI (device memory and streams only).

Every function checks shapes/dtypes/devices on the host before the launch and
passes raw device pointers plus ``torch.cuda.current_stream().cuda_stream``.
Outputs are allocated through torch's caching allocator; the kernels never
allocate.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

from . import _native as N

_DT = {torch.float16: N.OC_DTYPE_F16, torch.bfloat16: N.OC_DTYPE_BF16}


def _ptr(t: Optional[torch.Tensor]):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _stream(dev: torch.device):
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _need(t: torch.Tensor, name: str, dtype, shape=None, dev=None, align: int = 16):
    if not isinstance(t, torch.Tensor):
        raise TypeError(f"{name} must be a tensor")
    if t.device.type != "cuda":
        raise ValueError(f"{name} must be a CUDA/HIP device tensor, got {t.device}")
    if dev is not None and t.device != dev:
        raise ValueError(f"{name} is on {t.device}, expected {dev}")
    if dtype is not None and t.dtype not in (dtype if isinstance(dtype, tuple) else (dtype,)):
        raise TypeError(f"{name} must be {dtype}, got {t.dtype}")
    if shape is not None and tuple(t.shape) != tuple(shape):
        raise ValueError(f"{name} must have shape {tuple(shape)}, got {tuple(t.shape)}")
    if not t.is_contiguous():
        raise ValueError(f"{name} must be contiguous")
    if t.data_ptr() % align:
        raise ValueError(f"{name} must be {align}-byte aligned")


# ----------------------------------------------------------------- parity tools

def gptq_unpack_codes(qweight: torch.Tensor, bits: int) -> torch.Tensor:
    """codes [N, K] int32 (replaces unpack_int_weights, gptq_layer.py:142-157)."""
    _need(qweight, "qweight", torch.int32)
    k = qweight.shape[0] * 32 // bits
    n = qweight.shape[1]
    out = torch.empty((n, k), dtype=torch.int32, device=qweight.device)
    N.call("oc_gptq_unpack_codes", _ptr(qweight), k, n, bits, _ptr(out), _stream(qweight.device))
    return out


def gptq_unpack_zeros(qzeros: torch.Tensor, bits: int, out_features: int,
                      zero_format: int = N.OC_ZERO_RAW) -> torch.Tensor:
    """zeros [G, N] int32 (replaces unpack_zeros gptq_layer.py:173-184 + restore :550-557)."""
    _need(qzeros, "qzeros", torch.int32)
    g = qzeros.shape[0]
    out = torch.empty((g, out_features), dtype=torch.int32, device=qzeros.device)
    N.call("oc_gptq_unpack_zeros", _ptr(qzeros), g, out_features, bits, zero_format, _ptr(out),
           _stream(qzeros.device))
    return out


def gptq_dequant(qweight, qzeros, scales, g_idx, bits: int, group_size: int,
                 zero_format: int = N.OC_ZERO_V1, dtype=torch.float16) -> torch.Tensor:
    """W [N, K] in ``dtype``, bit-exact RNE(s * (q - z)) (gptq_layer.py:536-569)."""
    dev = qweight.device
    _need(qweight, "qweight", torch.int32)
    k, n = qweight.shape[0] * 32 // bits, qweight.shape[1]
    _need(scales, "scales", torch.float16, dev=dev)
    g = scales.shape[0]
    _need(qzeros, "qzeros", torch.int32, (g, n * bits // 32), dev)
    if g_idx is not None:
        _need(g_idx, "g_idx", torch.int32, (k,), dev)
    out = torch.empty((n, k), dtype=dtype, device=dev)
    N.call("oc_gptq_dequant", _ptr(qweight), _ptr(qzeros), _ptr(scales), _ptr(g_idx), k, n, g, bits,
           group_size, zero_format, _DT[dtype], _ptr(out), _stream(dev))
    return out


# ----------------------------------------------------------------- hot path

@dataclass
class PreparedGPTQ:
    """A layer repacked into the kernel layout (output of process_weights_after_loading)."""

    packed: torch.Tensor      # uint8 lane-chunk layout
    meta: torch.Tensor        # int32 [G, N_pad]: fp16 scale | restored zero << 16
    perm: Optional[torch.Tensor]  # int32 [K] or None (no act-order / identity)
    in_features: int
    out_features: int
    bits: int
    group_size: int
    num_groups: int
    _ws: dict = field(default_factory=dict, repr=False)  # workspace bytes per (M, plan generation)


def gptq_layout(k: int, n: int, bits: int):
    nbytes, kp, np_ = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
    N.call("oc_gptq_layout", k, n, bits, ctypes.byref(nbytes), ctypes.byref(kp), ctypes.byref(np_))
    return nbytes.value, kp.value, np_.value


def gptq_prepare(qweight, qzeros, scales, g_idx, bits: int, group_size: int,
                 zero_format: int = N.OC_ZERO_V1) -> PreparedGPTQ:
    """Repack checkpoint tensors (replaces vLLM's process_weights_after_loading)."""
    dev = qweight.device
    _need(qweight, "qweight", torch.int32)
    k, n = qweight.shape[0] * 32 // bits, qweight.shape[1]
    _need(scales, "scales", torch.float16, dev=dev)
    g = scales.shape[0]
    _need(qzeros, "qzeros", torch.int32, (g, n * bits // 32), dev)
    if g_idx is not None:
        _need(g_idx, "g_idx", torch.int32, (k,), dev)
    nbytes, _kp, n_pad = gptq_layout(k, n, bits)
    packed = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    meta = torch.empty((g, n_pad), dtype=torch.int32, device=dev)
    perm = torch.empty(k, dtype=torch.int32, device=dev) if g_idx is not None else None
    ident = ctypes.c_int(1)
    N.call("oc_gptq_prepare", _ptr(qweight), _ptr(qzeros), _ptr(scales), _ptr(g_idx), k, n, g, bits,
           group_size, zero_format, _ptr(packed), _ptr(meta), _ptr(perm), ctypes.byref(ident),
           _stream(dev))
    if ident.value:
        perm = None
    return PreparedGPTQ(packed, meta, perm, k, n, bits, group_size, g)


def gptq_gemm(x: torch.Tensor, prep: PreparedGPTQ, bias: Optional[torch.Tensor] = None,
              out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = x @ dequant(W)^T (+ bias) for x [..., K] (replaces GPTQLinearMethod.apply)."""
    dev = prep.packed.device
    if x.dtype not in _DT:
        raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
    k, n = prep.in_features, prep.out_features
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, layer expects {k}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    _need(x2, "x", x.dtype, dev=dev)
    m = x2.shape[0]
    if bias is not None:
        _need(bias, "bias", x.dtype, (n,), dev)
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=dev)
    else:
        _need(out, "out", x.dtype, (m, n), dev)
    key = (m, N.plan_generation())
    ws_bytes = prep._ws.get(key)
    if ws_bytes is None:
        ws_bytes = N.load().oc_gptq_workspace_bytes(m, k, n, prep.bits, prep.group_size,
                                                    int(prep.perm is not None))
        prep._ws[key] = ws_bytes
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    N.call("oc_gptq_gemm", _ptr(x2), m, k, n, _ptr(prep.packed), _ptr(prep.meta), _ptr(prep.perm),
           prep.bits, prep.group_size, _DT[x.dtype], _ptr(bias), _ptr(out), _ptr(ws), ws_bytes,
           _stream(dev))
    return out.reshape(*lead, n)


def gptq_gemm_noalloc(x: torch.Tensor, prep: PreparedGPTQ, bias: Optional[torch.Tensor] = None,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """gptq_gemm through oc_gptq_gemm_noalloc: the library's per-GPU scratch array instead of a
    workspace (nothing is allocated when ``out`` is given and x is contiguous)."""
    dev = prep.packed.device
    if x.dtype not in _DT:
        raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
    k, n = prep.in_features, prep.out_features
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, layer expects {k}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    _need(x2, "x", x.dtype, dev=dev)
    m = x2.shape[0]
    if bias is not None:
        _need(bias, "bias", x.dtype, (n,), dev)
    if out is None:
        out = torch.empty((m, n), dtype=x.dtype, device=dev)
    else:
        _need(out, "out", x.dtype, (m, n), dev)
    N.call("oc_gptq_gemm_noalloc", _ptr(x2), m, k, n, _ptr(prep.packed), _ptr(prep.meta), _ptr(prep.perm),
           prep.bits, prep.group_size, _DT[x.dtype], _ptr(bias), _ptr(out), _stream(dev))
    return out.reshape(*lead, n)


class OcGptqPart(ctypes.Structure):
    _fields_ = [("packed", ctypes.c_void_p), ("meta", ctypes.c_void_p), ("perm", ctypes.c_void_p),
                ("bias", ctypes.c_void_p), ("N", ctypes.c_int), ("bits", ctypes.c_int),
                ("group_size", ctypes.c_int)]


def gptq_gemm_grouped(x: torch.Tensor, preps: List[PreparedGPTQ],
                      biases: Optional[List[Optional[torch.Tensor]]] = None,
                      out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Parts of a fused module side by side: y[..., off_p:off_p+N_p] = x @ dequant(W_p)^T (+ b_p).

    The parts may differ in bits, group size and act-order (oc_gptq_gemm_grouped).
    """
    if not 1 <= len(preps) <= 8:
        raise ValueError(f"{len(preps)} parts; 1..8 are supported")
    dev = preps[0].packed.device
    if x.dtype not in _DT:
        raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
    k = preps[0].in_features
    if any(p.in_features != k for p in preps):
        raise ValueError("all parts of a fused module must have the same in_features")
    if x.shape[-1] != k:
        raise ValueError(f"x has {x.shape[-1]} features, layer expects {k}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    _need(x2, "x", x.dtype, dev=dev)
    m = x2.shape[0]
    n_total = sum(p.out_features for p in preps)
    if out is None:
        out = torch.empty((m, n_total), dtype=x.dtype, device=dev)
    else:
        _need(out, "out", x.dtype, (m, n_total), dev)
    arr = (OcGptqPart * len(preps))()
    for i, p in enumerate(preps):
        b = None if biases is None else biases[i]
        if b is not None:
            _need(b, "bias", x.dtype, (p.out_features,), dev)
        arr[i] = OcGptqPart(p.packed.data_ptr(), p.meta.data_ptr(), _ptr(p.perm), _ptr(b), p.out_features,
                            p.bits, p.group_size)
    ws_bytes = N.load().oc_gptq_grouped_workspace_bytes(arr, len(preps), m, k)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    N.call("oc_gptq_gemm_grouped", _ptr(x2), m, k, arr, len(preps), _DT[x.dtype], _ptr(out), n_total,
           _ptr(ws), ws_bytes, _stream(dev))
    return out.reshape(*lead, n_total)


# ---------------------------------------------------------------------------------- Hadamard

_HAD_BLOCKS: Dict = {}


def hadamard_order(n: int) -> int:
    """Block order the reference picks for n (hadamard_utils.py:79-175); raises where it asserts."""
    k = N.load().oc_hadamard_order(n)
    if k == 0:
        raise ValueError(f"no Hadamard decomposition n = K * 2^m for n={n}")
    return k


def hadamard_block(k: int, device) -> Optional[torch.Tensor]:
    """Device int8 [k, k] block (cached per device), None for k = 1."""
    if k == 1:
        return None
    key = (k, str(device))
    t = _HAD_BLOCKS.get(key)
    if t is None:
        host = (ctypes.c_int8 * (k * k))()
        N.call("oc_hadamard_block", k, host)
        t = torch.tensor(list(host), dtype=torch.int8).view(k, k).to(device)
        _HAD_BLOCKS[key] = t
    return t


_HAD_ROUNDING = {"fp32": N.OC_HAD_ROUND_FP32, "once": N.OC_HAD_ROUND_ONCE, "stages": N.OC_HAD_ROUND_STAGES}


def hadamard(x: torch.Tensor, out: Optional[torch.Tensor] = None, rounding: str = "stages") -> torch.Tensor:
    """Online Hadamard of the last axis: (H_K (x) H_L) x / sqrt(n), rounded as the reference's
    apply_online_hadamard (rotation.py:100-112) rounds: "fp32" for fp32_had=True (one rounding);
    for fp32_had=False "stages" (the reference's pure-PyTorch transform adds in x's dtype, every
    butterfly stage rounds; its default install) or "once" (with the fast_hadamard_transform
    package: the transform rounds once), each followed by the rounded 1/sqrt(n) division and the
    rounded H_K product."""
    if rounding not in _HAD_ROUNDING:
        raise ValueError(f"rounding must be one of {sorted(_HAD_ROUNDING)}, got {rounding!r}")
    if x.dtype not in _DT:
        raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
    n = x.shape[-1]
    k = hadamard_order(n)
    x2 = x.reshape(-1, n)
    if x2.stride(-1) != 1:
        x2 = x2.contiguous()
    if out is None:
        out = torch.empty_like(x2)
    blk = hadamard_block(k, x.device)
    # An output overlapping the input is written through a fresh buffer: the library serves
    # overlapping buffers with its one-workgroup-per-row kernel, whose fp32 summation order
    # differs from the small-M kernel's, and in-place calls should give the same bits.
    lo, hi = x2.data_ptr(), x2.data_ptr() + x2.shape[0] * x2.stride(0) * x2.element_size()
    olo, ohi = out.data_ptr(), out.data_ptr() + out.shape[0] * out.stride(0) * out.element_size()
    dst = torch.empty_like(x2) if (olo < hi and lo < ohi) else out
    N.call("oc_hadamard", _ptr(x2), x2.shape[0], n, x2.stride(0), _ptr(blk), k, _DT[x.dtype], _HAD_ROUNDING[rounding],
           _ptr(dst), dst.stride(0), _stream(x.device))
    if dst is not out:
        out.copy_(dst)
    return out.reshape(x.shape)
