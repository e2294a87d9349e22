"""Mixture-of-experts blocks with GPTQ experts, backed by ``oc_moe_gptq_forward``.

OneComp serves quantized MoE layers two ways:

- the HF path: ``_UnfusedExperts`` (onecomp/utils/unfuse_moe.py:33-114) holds
  one GPTQ ``gate_proj`` / ``up_proj`` / ``down_proj`` per expert and loops
  over the experts that the router hit, ``act_fn(gate) * up`` (or the gpt-oss
  ``combine_fn`` of :380-387), then ``index_add`` of the weighted outputs;
- vLLM: ``MixedGPTQConfig._get_moe_quant_method`` (vllm_plugins/gptq/
  vllm_plugin.py:240-283) hands the experts to vLLM's WNA16 fused-experts
  kernel (third-party, not installed here).

:func:`prepare_experts` repacks every expert once (gate|up merged per expert
into one layer, down separately) into two contiguous expert-major buffers;
:func:`moe_forward` runs the whole block as four launches with the expert of
each (token, slot) pair read on the device, so the router's output never
travels to the host.  :class:`GPTQExperts` is the HF-path drop-in with
``_UnfusedExperts``'s forward signature.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass
from typing import List, Optional, Sequence

import torch
from torch import nn

from . import _native as N
from .ops import _DT, _need, _ptr, _stream, gptq_layout

ACT_SILU, ACT_GELU_TANH, ACT_GPT_OSS = 0, 1, 2
_ACTS = {"silu": ACT_SILU, "swish": ACT_SILU, "gelu_pytorch_tanh": ACT_GELU_TANH, "gelu_tanh": ACT_GELU_TANH,
         "gpt_oss": ACT_GPT_OSS}


@dataclass
class PreparedExperts:
    w13: torch.Tensor      # uint8 [E, stride13]: merged gate|up (H -> 2I), gate columns first
    meta13: torch.Tensor   # int32 [E, G13 * N_pad(2I)]
    b13: Optional[torch.Tensor]  # [E, 2I] or None
    w2: torch.Tensor       # uint8 [E, stride2]: down (I -> H)
    meta2: torch.Tensor    # int32 [E, G2 * N_pad(H)]
    b2: Optional[torch.Tensor]   # [E, H] or None
    num_experts: int
    hidden: int
    inter: int
    bits: int
    group_size: int
    perm13: Optional[torch.Tensor] = None  # int32 [E, H]: act-order gate|up k order, or None
    perm2: Optional[torch.Tensor] = None   # int32 [E, I]: act-order down k order, or None


def _prepare_into(qweight, qzeros, scales, bits, group_size, zero_format, packed, meta, g_idx=None, perm=None):
    """Repack one expert's layer; with g_idx (act-order) its k order goes to ``perm``.  Returns True
    when the order is the identity."""
    k, n = qweight.shape[0] * 32 // bits, qweight.shape[1]
    g = scales.shape[0]
    ident = ctypes.c_int(1)
    gi = None if g_idx is None else g_idx.to(torch.int32).contiguous()
    N.call("oc_gptq_prepare", _ptr(qweight), _ptr(qzeros), _ptr(scales), _ptr(gi), k, n, g, bits, group_size,
           zero_format, _ptr(packed), _ptr(meta), _ptr(perm), ctypes.byref(ident), _stream(qweight.device))
    return bool(ident.value)


def _prepare(E, H, I, bits, group_size, zero_format, w13_of, w2_of, b13, b2, dev, g13_of=None,
             g2_of=None) -> PreparedExperts:
    if I * bits % 32:
        raise ValueError(f"intermediate size {I} x {bits} bits does not pack the merged gate|up zeros")
    nb13, _, np13 = gptq_layout(H, 2 * I, bits)
    nb2, _, np2 = gptq_layout(I, H, bits)
    gs13 = group_size if group_size > 0 else H
    gs2 = group_size if group_size > 0 else I
    g13, g2 = (H + gs13 - 1) // gs13, (I + gs2 - 1) // gs2
    w13 = torch.empty((E, nb13), dtype=torch.uint8, device=dev)
    meta13 = torch.empty((E, g13 * np13), dtype=torch.int32, device=dev)
    w2 = torch.empty((E, nb2), dtype=torch.uint8, device=dev)
    meta2 = torch.empty((E, g2 * np2), dtype=torch.int32, device=dev)
    perm13 = torch.empty((E, H), dtype=torch.int32, device=dev) if g13_of is not None else None
    perm2 = torch.empty((E, I), dtype=torch.int32, device=dev) if g2_of is not None else None
    ident13 = ident2 = True
    for e in range(E):
        qw, qz, sc = w13_of(e)
        _need(qw, "gate|up qweight", torch.int32, dev=dev)
        ident13 &= _prepare_into(qw.contiguous(), qz.contiguous(), sc.to(torch.float16).contiguous(), bits,
                                 group_size, zero_format, w13[e], meta13[e],
                                 None if perm13 is None else g13_of(e), None if perm13 is None else perm13[e])
        qw, qz, sc = w2_of(e)
        _need(qw, "down qweight", torch.int32, dev=dev)
        ident2 &= _prepare_into(qw.contiguous(), qz.contiguous(), sc.to(torch.float16).contiguous(), bits,
                                group_size, zero_format, w2[e], meta2[e],
                                None if perm2 is None else g2_of(e), None if perm2 is None else perm2[e])
    # every expert in checkpoint order: no gathers at run time
    return PreparedExperts(w13, meta13, b13, w2, meta2, b2, E, H, I, bits, group_size,
                           None if ident13 else perm13, None if ident2 else perm2)


def prepare_experts(gate: Sequence, up: Sequence, down: Sequence, bits: int, group_size: int,
                    zero_format: int = N.OC_ZERO_V1, gate_up_bias: Optional[Sequence] = None,
                    down_bias: Optional[Sequence] = None) -> PreparedExperts:
    """gate / up / down: per expert (qweight, qzeros, scales[, g_idx]) in the AutoGPTQ layout on the
    device; g_idx (act-order) is optional, and gate and up of one expert must share it (their
    input and its calibration statistics are the same; the merged gate|up layer has one k order).

    All experts share bits and group size (vllm_plugin.py:220-239 relies on the same).  Biases:
    per expert gate|up [2I] (gate first) and down [H].
    """
    E = len(gate)
    if not (E == len(up) == len(down)) or E == 0:
        raise ValueError("gate, up and down need one entry per expert")
    dev = gate[0][0].device
    H = gate[0][0].shape[0] * 32 // bits
    I = gate[0][0].shape[1]

    def w13_of(e):
        (gq, gz, gsc), (uq, uz, usc) = gate[e][:3], up[e][:3]
        return torch.cat([gq, uq], dim=1), torch.cat([gz, uz], dim=1), torch.cat([gsc, usc], dim=1)

    def gidx(t):
        return t[3] if len(t) > 3 and t[3] is not None else None

    act13 = any(gidx(t) is not None for t in list(gate) + list(up))
    act2 = any(gidx(t) is not None for t in down)
    g13 = g2 = None
    if act13:  # checked for every expert before anything is repacked
        g13 = []
        for e in range(E):
            gg, ug = gidx(gate[e]), gidx(up[e])
            if gg is None or ug is None or not torch.equal(gg.to(torch.int32), ug.to(torch.int32)):
                raise ValueError(f"expert {e}: act-order gate_proj and up_proj need the same g_idx "
                                 "(the merged gate|up layer has one k order)")
            g13.append(gg)
    if act2:
        g2 = []
        for e in range(E):
            if gidx(down[e]) is None:
                raise ValueError(f"expert {e}: down_proj has no g_idx while other experts' do")
            g2.append(gidx(down[e]))
    g13_of = None if g13 is None else (lambda e: g13[e])
    g2_of = None if g2 is None else (lambda e: g2[e])
    b13 = None if gate_up_bias is None else torch.stack([b.reshape(-1) for b in gate_up_bias]).contiguous()
    b2 = None if down_bias is None else torch.stack([b.reshape(-1) for b in down_bias]).contiguous()
    return _prepare(E, H, I, bits, group_size, zero_format, w13_of, lambda e: down[e][:3], b13, b2, dev,
                    g13_of, g2_of)


def prepare_experts_merged(w13_qweight: torch.Tensor, w13_qzeros: torch.Tensor, w13_scales: torch.Tensor,
                           w2_qweight: torch.Tensor, w2_qzeros: torch.Tensor, w2_scales: torch.Tensor, bits: int,
                           group_size: int, zero_format: int = N.OC_ZERO_V1, w13_bias: Optional[torch.Tensor] = None,
                           w2_bias: Optional[torch.Tensor] = None, w13_g_idx: Optional[torch.Tensor] = None,
                           w2_g_idx: Optional[torch.Tensor] = None) -> PreparedExperts:
    """Expert-stacked AutoGPTQ tensors of a FusedMoE layer: w13_* [E, ...] hold each expert's gate
    and up side by side (gate columns first), w2_* its down; biases [E, 2I] and [E, H] or None;
    act-order g_idx [E, H] (gate|up) and [E, I] (down) or None."""
    E = w13_qweight.shape[0]
    H = w13_qweight.shape[1] * 32 // bits
    I = w13_qweight.shape[2] // 2
    return _prepare(E, H, I, bits, group_size, zero_format,
                    lambda e: (w13_qweight[e], w13_qzeros[e], w13_scales[e]),
                    lambda e: (w2_qweight[e], w2_qzeros[e], w2_scales[e]),
                    None if w13_bias is None else w13_bias.contiguous(),
                    None if w2_bias is None else w2_bias.contiguous(), w13_qweight.device,
                    None if w13_g_idx is None else (lambda e: w13_g_idx[e]),
                    None if w2_g_idx is None else (lambda e: w2_g_idx[e]))


def moe_forward(x: torch.Tensor, top_k_index: torch.Tensor, top_k_weights: torch.Tensor, ex: PreparedExperts,
                act: str = "silu", alpha: float = 1.702, limit: float = 7.0,
                router_weight_on_input: bool = False) -> torch.Tensor:
    """y[t] = sum_j w[t, j] * down_e(act(gate_e(x[t]), up_e(x[t]))), e = top_k_index[t, j].

    router_weight_on_input (vLLM's apply_router_weight_on_input, top-1 routing only): the experts
    run on x[t] * w[t] (rounded to x's dtype, as vLLM scales the hidden states) and their outputs
    are summed unweighted."""
    if x.dtype not in _DT:
        raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
    if act not in _ACTS:
        raise ValueError(f"unknown activation {act!r}; one of {sorted(_ACTS)}")
    lead = x.shape[:-1]
    x2 = x.reshape(-1, ex.hidden)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    topk = top_k_index.shape[-1]
    ids = top_k_index.reshape(m, topk).to(torch.int32).contiguous()
    w = top_k_weights.reshape(m, topk).to(torch.float32).contiguous()
    if router_weight_on_input:
        if topk != 1:
            raise ValueError(f"router weights on the input need top-1 routing, got top-{topk}")
        x2 = (x2 * top_k_weights.reshape(m, 1).to(x2.dtype)).contiguous()
        w = torch.ones_like(w)
    dt = x.dtype
    b13 = None if ex.b13 is None else ex.b13.to(dt)
    b2 = None if ex.b2 is None else ex.b2.to(dt)
    y = torch.empty((m, ex.hidden), dtype=dt, device=x.device)
    act_order = ex.perm13 is not None or ex.perm2 is not None
    nbytes = N.load().oc_moe_workspace_bytes(m, ex.hidden, ex.inter, topk, int(act_order))
    ws = torch.empty(max(nbytes, 1), dtype=torch.uint8, device=x.device)
    N.call("oc_moe_gptq_forward", _ptr(x2), m, ex.hidden, ex.inter, ex.num_experts, topk, _ptr(ids), _ptr(w),
           _ptr(ex.w13), ex.w13.shape[1], _ptr(ex.meta13), ex.meta13.shape[1], _ptr(b13), _ptr(ex.w2),
           ex.w2.shape[1], _ptr(ex.meta2), ex.meta2.shape[1], _ptr(b2), _ptr(ex.perm13), _ptr(ex.perm2), ex.bits,
           ex.group_size, _ACTS[act],
           float(alpha), float(limit), _DT[dt], _ptr(y), _ptr(ws), nbytes, _stream(x.device))
    return y.reshape(*lead, ex.hidden)


class GPTQExperts(nn.Module):
    """Drop-in for ``_UnfusedExperts`` (unfuse_moe.py:33-114) whose experts hold GPTQ
    ``gate_proj`` / ``up_proj`` / ``down_proj`` layers (``hf.GPTQLinear`` or any module with the
    AutoGPTQ buffers ``qweight`` / ``qzeros`` / ``scales`` and attributes ``wbits`` /
    ``groupsize``).  ``act``: ``"silu"`` or ``"gelu_pytorch_tanh"`` for ``act_fn(gate) * up``,
    ``"gpt_oss"`` for the gpt-oss combine with ``alpha`` / ``limit``."""

    def __init__(self, num_experts: int, experts: List[nn.Module], act: str = "silu",
                 alpha: float = 1.702, limit: float = 7.0):
        super().__init__()
        self._num_experts = num_experts
        for i, expert in enumerate(experts):
            self.add_module(str(i), expert)
        self.act, self.alpha, self.limit = act, alpha, limit
        self._prep = None
        self._stamp = None

    def __len__(self):
        return self._num_experts

    def __getitem__(self, idx):
        return getattr(self, str(int(idx)))

    def __iter__(self):
        return iter(self._modules.values())

    def _prepared(self) -> PreparedExperts:
        lins = [(e.gate_proj, e.up_proj, e.down_proj) for e in self]
        tensors = [t for trio in lins for lin in trio for t in (lin.qweight, lin.qzeros, lin.scales,
                                                                 getattr(lin, "g_idx", None)) if t is not None]
        stamp = tuple((t.data_ptr(), t._version) for t in tensors)
        if self._prep is None or stamp != self._stamp:
            bits = lins[0][0].wbits
            gs = lins[0][0].groupsize if lins[0][0].groupsize and lins[0][0].groupsize > 0 else -1
            for trio in lins:
                for lin in trio:
                    if lin.wbits != bits or (lin.groupsize if lin.groupsize and lin.groupsize > 0 else -1) != gs:
                        raise ValueError("all experts of a GPTQExperts block need the same bits and group size")
            fmt = N.OC_ZERO_V2 if getattr(lins[0][0], "checkpoint_format", "gptq") == "gptq_v2" else N.OC_ZERO_V1
            has_b = lins[0][0].bias is not None
            gub = [torch.cat([g.bias, u.bias]) for g, u, _ in lins] if has_b else None
            db = [d.bias for _, _, d in lins] if lins[0][2].bias is not None else None
            def gi(lin):  # act-order layers carry their g_idx
                return getattr(lin, "g_idx", None) if getattr(lin, "actorder", False) else None

            self._prep = prepare_experts([(g.qweight, g.qzeros, g.scales, gi(g)) for g, _, _ in lins],
                                         [(u.qweight, u.qzeros, u.scales, gi(u)) for _, u, _ in lins],
                                         [(d.qweight, d.qzeros, d.scales, gi(d)) for _, _, d in lins], bits, gs, fmt,
                                         gub, db)
            self._stamp = stamp
        return self._prep

    def forward(self, hidden_states: torch.Tensor, top_k_index: Optional[torch.Tensor] = None,
                top_k_weights: Optional[torch.Tensor] = None, router_indices: Optional[torch.Tensor] = None,
                routing_weights: Optional[torch.Tensor] = None) -> torch.Tensor:
        # the two router argument conventions of unfuse_moe.py:61-76
        if top_k_index is None:
            top_k_index = router_indices
        if top_k_weights is None:
            top_k_weights = routing_weights
        if hidden_states.device.type != "cuda":
            raise RuntimeError("GPTQExperts (onecomp-amd) runs on a HIP device")
        return moe_forward(hidden_states, top_k_index, top_k_weights, self._prepared(), self.act, self.alpha,
                           self.limit)
