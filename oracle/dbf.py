"""DBF / MDBF oracle: sign packing, rank formula and forwards (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restates (reference = /root/reference, read as text, never imported):

- ``pack_binary``                     onecomp/quantizer/dbf/dbf_layer.py:32-44
- ``unpack_binary`` / ``_factor``     dbf_layer.py:47-52, :71-86
- ``unpack_sign_bits``                vllm_plugins/dbf/modules/naive.py:9-42
- rank ``_compute_mid_features``      vllm_plugins/dbf/vllm_plugin.py:81-83
- per-part sizes / offsets            vllm_plugin.py:118-152
- 5-stage forward                     vllm_plugin.py:275-294, dbf_layer.py:251-268
- fused parts + bias                  vllm_plugin.py:330-381, :414-418
- MDBF factors and forward            onecomp/quantizer/mdbf/mdbf_layer.py:278-290, :338-344
- MDBF P-path sum                     mdbf_layer.py:412-420

Sign layout: element e of a flattened row-major R x C factor is bit
``7 - (e % 8)`` of byte ``e // 8``; bit 1 -> +1, bit 0 -> -1; trailing
padding bits are 1.
"""

from __future__ import annotations

import numpy as np

from .gptq import f32_to_bf16_bits, to_f32


def pack_binary(signs: np.ndarray) -> np.ndarray:
    """±1 (any shape) -> uint8 [ceil(numel/8)], MSB first (dbf_layer.py:32-44).

    Zero counts as +1 (``x >= 0``); padding bits are 1.
    """
    flat = (np.asarray(signs).reshape(-1) >= 0).astype(np.uint8)
    pad = (-flat.size) % 8
    if pad:
        flat = np.concatenate([flat, np.ones(pad, dtype=np.uint8)])
    flat = flat.reshape(-1, 8)
    out = np.zeros(flat.shape[0], dtype=np.uint8)
    for i in range(8):
        out |= (flat[:, i] << (7 - i)).astype(np.uint8)
    return out


def unpack_binary(packed: np.ndarray) -> np.ndarray:
    """uint8 [B] -> int8 ±1 [8B] (dbf_layer.py:47-52, naive.py:27-35)."""
    p = np.asarray(packed, dtype=np.uint8)
    bits = np.empty((p.size, 8), dtype=np.int8)
    for i in range(8):
        bits[:, i] = (p >> (7 - i)) & 1
    return bits.reshape(-1) * 2 - 1


def unpack_binary_factor(packed: np.ndarray, shape) -> np.ndarray:
    """uint8 buffer -> int8 ±1 [rows, cols] (dbf_layer.py:71-86, naive.py:37-42)."""
    rows, cols = int(shape[0]), int(shape[1])
    return unpack_binary(packed)[: rows * cols].reshape(rows, cols)


def mid_features(bits: float, in_features: int, out_features: int) -> int:
    """DBF rank r = min(min(K, N), int(bits*K*N/(K+N))) (vllm_plugin.py:81-83)."""
    r = int(bits * (in_features * out_features) / (in_features + out_features))
    return min(min(in_features, out_features), r)


def part_layout(bits: float, in_features: int, out_sizes):
    """Per-part mid sizes, bp1/bp3 byte sizes and offsets (vllm_plugin.py:118-152)."""
    mids = [mid_features(bits, in_features, n) for n in out_sizes]
    bp1 = [(r * in_features + 7) // 8 for r in mids]
    bp3 = [(n * r + 7) // 8 for n, r in zip(out_sizes, mids)]

    def offs(sizes):
        o, c = [], 0
        for s in sizes:
            o.append(c)
            c += s
        return o

    return {
        "mid_sizes": mids,
        "bp1_sizes": bp1,
        "bp3_sizes": bp3,
        "scaling2_offsets": offs(mids),
        "scaling4_offsets": offs(list(out_sizes)),
        "bp1_offsets": offs(bp1),
        "bp3_offsets": offs(bp3),
    }


def _round(v: np.ndarray, dtype: str) -> np.ndarray:
    v32 = np.asarray(v, dtype=np.float32)
    if dtype in ("bf16", "bfloat16"):
        return to_f32(f32_to_bf16_bits(v32), "bf16")
    if dtype in ("fp16", "float16", "half"):
        return v32.astype(np.float16).astype(np.float32)
    return v32


def dbf_forward(x, s0, bp1, s2, bp3, s4, in_features, mid, out_features,
                dtype="fp16", staged=False, bias=None) -> np.ndarray:
    """y = s4 * (S1 @ (s2 * (S2 @ (s0 * x)))) (+ bias), fp32 result.

    vllm_plugin.py:275-294 / dbf_layer.py:251-268.  S2 = bp1 unpacked to
    [mid, K]; S1 = bp3 unpacked to [N, mid].  With ``staged=True`` every
    stage is rounded to the activation dtype as the reference does; otherwise
    everything stays in float64 (the fp32-accumulated target).
    """
    S2 = unpack_binary_factor(bp1, (mid, in_features)).astype(np.float64)
    S1 = unpack_binary_factor(bp3, (out_features, mid)).astype(np.float64)
    xf = to_f32(x, dtype).astype(np.float64)
    rnd = (lambda v: _round(v, dtype).astype(np.float64)) if staged else (lambda v: v)
    f = lambda v: to_f32(v, dtype).astype(np.float64)  # noqa: E731
    h = rnd(xf * f(s0))
    h = rnd(h @ S2.T)
    h = rnd(h * f(s2))
    h = rnd(h @ S1.T)
    h = rnd(h * f(s4))
    if bias is not None:
        h = rnd(h + f(bias))
    return h.astype(np.float32)


def dbf_dense_weight(s0, bp1, s2, bp3, s4, in_features, mid, out_features) -> np.ndarray:
    """Dense W = diag(s4) S1 diag(s2) S2 diag(s0) in float64.

    The closed form behind the identity-forward reconstruction of
    onecomp/cpu/export/dequantize.py:40-77.
    """
    S2 = unpack_binary_factor(bp1, (mid, in_features)).astype(np.float64)
    S1 = unpack_binary_factor(bp3, (out_features, mid)).astype(np.float64)
    a = np.asarray(s4, dtype=np.float64)
    m = np.asarray(s2, dtype=np.float64)
    b = np.asarray(s0, dtype=np.float64)
    return a[:, None] * (S1 @ (m[:, None] * S2)) * b[None, :]


def mdbf_path_factors(a_packed, a_shape, b_packed, b_shape, a_amp, b_amp, qu_amp, qv_amp,
                      dtype="fp16"):
    """F = S_A * (A_amp @ Q_U^T), G = S_B * (Q_V @ B_amp^T) in the activation dtype.

    mdbf_layer.py:278-290.  S_A is [n, r], S_B is [r, m]; amps are [*, l].
    The amp products are rounded to ``dtype`` as the reference does.
    """
    SA = unpack_binary_factor(a_packed, a_shape).astype(np.float32)
    SB = unpack_binary_factor(b_packed, b_shape).astype(np.float32)
    amp_a = _round(_round(a_amp, dtype) @ _round(qu_amp, dtype).T, dtype)
    amp_b = _round(_round(qv_amp, dtype) @ _round(b_amp, dtype).T, dtype)
    return _round(SA * amp_a, dtype), _round(SB * amp_b, dtype)


def mdbf_forward(x, paths, dtype="fp16", bias=None) -> np.ndarray:
    """y = sum_p (x @ G_p^T) @ F_p^T (+ bias), float64 accumulation, fp32 result.

    mdbf_layer.py:338-344 (per path) and :412-420 (sum over P paths).  Each
    ``paths`` entry is a dict with keys A_sign_packed, A_shape, B_sign_packed,
    B_shape, A_amp, B_amp, Q_U_amp, Q_V_amp.
    """
    xf = to_f32(x, dtype).astype(np.float64)
    y = None
    for p in paths:
        F, G = mdbf_path_factors(p["A_sign_packed"], p["A_shape"], p["B_sign_packed"],
                                 p["B_shape"], p["A_amp"], p["B_amp"], p["Q_U_amp"],
                                 p["Q_V_amp"], dtype)
        yp = (xf @ G.astype(np.float64).T) @ F.astype(np.float64).T
        y = yp if y is None else y + yp
    if bias is not None:
        y = y + to_f32(bias, dtype).astype(np.float64)
    return y.astype(np.float32)
