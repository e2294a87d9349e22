"""CPU restatement of OneComp's unfused MoE forward over GPTQ experts (test infrastructure only:
imported by tests/, never by the product path).

- ``moe_forward`` follows ``_UnfusedExperts.forward`` (onecomp/utils/unfuse_moe.py:61-114): for
  every expert the router hit (ascending id), gate / up of its tokens (rounded to the activation
  dtype, as the fp16 linears round), ``act_fn(gate) * up`` or the gpt-oss ``combine_fn``
  (:380-387), down (rounded), times the routing weight (rounded), then ``index_add`` into an
  activation-dtype output in that order.
- ``gpt_oss_combine`` restates ``_gpt_oss_combine_gate_up`` (:380-387) with each torch op's
  rounding to the activation dtype.
"""

from __future__ import annotations

import numpy as np

from . import gptq as og


def _r(v, dtype):
    """Round float32 values to the activation dtype and return them as float32."""
    v = np.asarray(v, dtype=np.float32)
    if dtype == "bf16":
        return og.bf16_bits_to_f32(og.f32_to_bf16_bits(v))
    return v.astype(np.float16).astype(np.float32)


def silu(g, dtype):
    g = np.asarray(g, dtype=np.float32)
    return _r(g / (1.0 + np.exp(-g)), dtype)


def gelu_tanh(g, dtype):
    g = np.asarray(g, dtype=np.float32)
    return _r(0.5 * g * (1.0 + np.tanh(0.7978845608028654 * (g + 0.044715 * g ** 3))), dtype)


def gpt_oss_combine(gate, up, alpha, limit, dtype):
    """(up.clamp(-limit, limit) + 1) * (g * sigmoid(g * alpha)), g = gate.clamp(max=limit)."""
    g = np.minimum(np.asarray(gate, np.float32), np.float32(limit))
    u = np.clip(np.asarray(up, np.float32), -np.float32(limit), np.float32(limit))
    ga = _r(g * np.float32(alpha), dtype)
    sig = _r(1.0 / (1.0 + np.exp(-ga)), dtype)
    glu = _r(g * sig, dtype)
    return _r(_r(u + 1.0, dtype) * glu, dtype)


def moe_forward(x, top_k_index, top_k_weights, experts, act="silu", alpha=1.702, limit=7.0, dtype="fp16"):
    """experts: per expert dict(gate=W [I, H], up=W [I, H], down=W [H, I]) dequantised fp32 (exact
    values of the activation-dtype weights), optional gate_bias/up_bias [I], down_bias [H].
    x: [M, H] float32 values of activation-dtype numbers; returns [M, H] float32 (rounded)."""
    x = np.asarray(x, np.float32)
    idx = np.asarray(top_k_index)
    wts = _r(np.asarray(top_k_weights, np.float32), dtype)
    out = np.zeros_like(x)
    for e in sorted(set(int(v) for v in idx.reshape(-1))):
        if e < 0 or e >= len(experts):
            continue
        tok, pos = np.nonzero(idx == e)
        ex = experts[e]
        xs = x[tok].astype(np.float64)
        gate = _r(xs @ ex["gate"].T.astype(np.float64) + ex.get("gate_bias", 0.0), dtype)
        up = _r(xs @ ex["up"].T.astype(np.float64) + ex.get("up_bias", 0.0), dtype)
        if act == "gpt_oss":
            h = gpt_oss_combine(gate, up, alpha, limit, dtype)
        else:
            a = silu(gate, dtype) if act == "silu" else gelu_tanh(gate, dtype)
            h = _r(a * up, dtype)
        d = _r(h.astype(np.float64) @ ex["down"].T.astype(np.float64) + ex.get("down_bias", 0.0), dtype)
        d = _r(d * wts[tok, pos][:, None], dtype)
        for row, t in enumerate(tok):  # index_add_ in the activation dtype, in token order
            out[t] = _r(out[t] + d[row], dtype)
    return out
