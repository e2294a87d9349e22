"""GPTQ oracle: AutoGPTQ packing, zero restore, g_idx and dequantisation (numpy).

TEST INFRASTRUCTURE ONLY -- see ``oracle/__init__.py``.

Restates (reference = /root/reference, read as text, never imported):

- ``_pack_rows`` / ``_unpack_rows``        onecomp/quantizer/gptq/gptq_layer.py:36-126
- ``pack_int_weights`` / ``unpack_int_weights``  gptq_layer.py:129-157
- ``pack_zeros`` / ``unpack_zeros``        gptq_layer.py:160-184
- v1/v2 zero restore                      gptq_layer.py:543-557, onecomp/cpu/export/checkpoint.py:217-221
- ``g_idx`` construction                  gptq_layer.py:423-433, checkpoint.py:223-232
- dequant ``scale * (q - zero)``          gptq_layer.py:559-566, checkpoint.py:249-259
- cast to activation dtype + F.linear     gptq_layer.py:568-572

Conventions: codes Q are [N, K] (out, in) int32; ``qweight`` is [K*b/32, N]
int32; ``qzeros`` is [G, N*b/32] int32; ``scales`` is [G, N] fp16.  bf16
values are carried as uint16 bit patterns (numpy has no bf16 dtype).
"""

from __future__ import annotations

import numpy as np

SUPPORTED_BITS = (2, 3, 4, 8)


def _check_bits(bits: int) -> None:
    if bits not in SUPPORTED_BITS:
        raise ValueError(f"Unsupported wbits: {bits}")


def _slot_layout_3bit():
    """(word, offset, first_bits) of each of the 32 codes in a 96-bit block.

    gptq_layer.py:64-81 (pack) and :109-124 (unpack): code j starts at bit 3j
    of a little-endian 3-word stream; slots 10 (offset 30) and 21 (offset 31)
    straddle two words.
    """
    out = []
    for j in range(32):
        start = 3 * j
        out.append((start // 32, start % 32, min(3, 32 - start % 32)))
    return out


def pack_rows(matrix: np.ndarray, bits: int) -> np.ndarray:
    """Pack integer rows along dim 0 into int32 words (gptq_layer.py:36-83).

    Values are masked to ``bits`` first (gptq_layer.py:51), so a v1 ``-1``
    zero stores as ``2^bits - 1`` and never corrupts a neighbouring slot.
    """
    _check_bits(bits)
    m = np.asarray(matrix).astype(np.int64) & ((1 << bits) - 1)
    m = m.astype(np.uint32)
    rows, cols = m.shape
    if bits in (2, 4, 8):
        pf = 32 // bits
        if rows % pf:
            raise ValueError(f"rows ({rows}) must be divisible by pack_factor ({pf})")
        r = m.reshape(rows // pf, pf, cols)
        packed = np.zeros((rows // pf, cols), dtype=np.uint32)
        for i in range(pf):
            packed |= r[:, i, :] << np.uint32(i * bits)
        return packed.view(np.int32)
    if rows % 32:
        raise ValueError(f"rows ({rows}) must be divisible by 32 for 3-bit packing")
    nb = rows // 32
    r = m.reshape(nb, 32, cols)
    packed = np.zeros((nb, 3, cols), dtype=np.uint32)
    for j, (w, off, first) in enumerate(_slot_layout_3bit()):
        v = r[:, j, :]
        if first == 3:
            packed[:, w, :] |= v << np.uint32(off)
        else:
            packed[:, w, :] |= (v & np.uint32((1 << first) - 1)) << np.uint32(off)
            packed[:, w + 1, :] |= v >> np.uint32(first)
    return packed.reshape(nb * 3, cols).view(np.int32)


def unpack_rows(packed: np.ndarray, bits: int, num_rows: int) -> np.ndarray:
    """Unpack int32 words along dim 0 (gptq_layer.py:86-126) -> int32 codes."""
    _check_bits(bits)
    p = np.ascontiguousarray(packed).view(np.uint32)
    prow, cols = p.shape
    mask = np.uint32((1 << bits) - 1)
    if bits in (2, 4, 8):
        pf = 32 // bits
        out = np.empty((prow, pf, cols), dtype=np.uint32)
        for i in range(pf):
            out[:, i, :] = (p >> np.uint32(i * bits)) & mask
        return out.reshape(prow * pf, cols)[:num_rows].astype(np.int32)
    nb = prow // 3
    p3 = p.reshape(nb, 3, cols)
    out = np.empty((nb, 32, cols), dtype=np.uint32)
    for j, (w, off, first) in enumerate(_slot_layout_3bit()):
        if first == 3:
            out[:, j, :] = (p3[:, w, :] >> np.uint32(off)) & mask
        else:
            lo = (p3[:, w, :] >> np.uint32(off)) & np.uint32((1 << first) - 1)
            hi = p3[:, w + 1, :] & np.uint32((1 << (3 - first)) - 1)
            out[:, j, :] = lo | (hi << np.uint32(first))
    return out.reshape(nb * 32, cols)[:num_rows].astype(np.int32)


def pack_int_weights(codes_nk: np.ndarray, bits: int) -> np.ndarray:
    """Q [N, K] -> qweight [K*b/32, N] (gptq_layer.py:129-139)."""
    return pack_rows(np.ascontiguousarray(np.asarray(codes_nk).T), bits)


def unpack_int_weights(qweight: np.ndarray, bits: int, shape_nk) -> np.ndarray:
    """qweight [K*b/32, N] -> Q [N, K] (gptq_layer.py:142-157)."""
    k = shape_nk[1]
    return np.ascontiguousarray(unpack_rows(qweight, bits, k).T)


def pack_zeros(zeros_gn: np.ndarray, bits: int) -> np.ndarray:
    """Zs [G, N] -> qzeros [G, N*b/32], packed along N (gptq_layer.py:160-170)."""
    return np.ascontiguousarray(pack_rows(np.ascontiguousarray(np.asarray(zeros_gn).T), bits).T)


def unpack_zeros(qzeros: np.ndarray, bits: int, out_features: int) -> np.ndarray:
    """qzeros [G, N*b/32] -> Zs [G, N] (gptq_layer.py:173-184)."""
    return np.ascontiguousarray(
        unpack_rows(np.ascontiguousarray(np.asarray(qzeros).T), bits, out_features).T
    )


def restore_zeros(zs: np.ndarray, bits: int, checkpoint_format: str = "gptq") -> np.ndarray:
    """Stored zero fields -> zero points (gptq_layer.py:543-557, checkpoint.py:217-221).

    v1 (any format other than ``"gptq_v2"``) is modular: ``(Zs + 1) & (2^b-1)``,
    so a stored ``2^b - 1`` (raw zero 0) wraps to 0.  v2 keeps ``Zs``.
    """
    zs = np.asarray(zs).astype(np.int32)
    if checkpoint_format != "gptq_v2":
        return (zs + 1) & ((1 << bits) - 1)
    return zs


def g_idx_from_perm(perm: np.ndarray, group_size: int) -> np.ndarray:
    """Act-order g_idx = argsort(perm) // gs (gptq_layer.py:423-428)."""
    invperm = np.argsort(np.asarray(perm), kind="stable")
    return (invperm // group_size).astype(np.int32)


def default_g_idx(in_features: int, group_size: int) -> np.ndarray:
    """g_idx without act-order (gptq_layer.py:429-432): k // gs, or 0 for gs = -1."""
    if group_size == -1:
        return np.zeros(in_features, dtype=np.int32)
    return (np.arange(in_features) // group_size).astype(np.int32)


def dequant_fp32(codes_nk, scales_gn, zeros_gn, g_idx) -> np.ndarray:
    """W32[n, k] = fp32(s[g_idx[k], n]) * fp32(q[n, k] - z[g_idx[k], n]).

    gptq_layer.py:559-566 and checkpoint.py:249-259.  The product of an fp16
    scale (11-bit significand) and an integer |q - z| <= 255 is exact in fp32,
    so this value is the exact real product.
    """
    g = np.asarray(g_idx).astype(np.int64)
    s = np.asarray(scales_gn).astype(np.float32)[g, :].T
    z = np.asarray(zeros_gn).astype(np.float32)[g, :].T
    return s * (np.asarray(codes_nk).astype(np.float32) - z)


def f32_to_bf16_bits(x: np.ndarray) -> np.ndarray:
    """fp32 -> bf16 with IEEE round-to-nearest-even, as uint16 bit patterns.

    Matches torch's ``Tensor.to(torch.bfloat16)`` on finite inputs (pinned in
    tests against torch).  NaN is kept quiet.
    """
    u = np.ascontiguousarray(np.asarray(x, dtype=np.float32)).view(np.uint32).astype(np.uint64)
    bias = ((u >> 16) & 1) + 0x7FFF
    r = ((u + bias) >> 16).astype(np.uint16)
    nan = np.isnan(np.asarray(x, dtype=np.float32))
    if nan.any():
        r = np.where(nan, ((u >> 16) | 0x40).astype(np.uint16), r)
    return r


def bf16_bits_to_f32(b: np.ndarray) -> np.ndarray:
    return (np.asarray(b).astype(np.uint32) << 16).view(np.float32)


def round_to(w32: np.ndarray, dtype: str) -> np.ndarray:
    """Cast fp32 -> activation dtype, one RNE rounding (gptq_layer.py:568-569).

    Returns fp16 values (``np.float16``) or bf16 bit patterns (``np.uint16``).
    """
    if dtype in ("fp16", "float16", "half"):
        return np.asarray(w32, dtype=np.float32).astype(np.float16)
    if dtype in ("bf16", "bfloat16"):
        return f32_to_bf16_bits(w32)
    raise ValueError(f"unsupported dtype {dtype}")


def dequantize(qweight, qzeros, scales, g_idx, bits: int, checkpoint_format="gptq", dtype="fp16"):
    """Checkpoint tensors -> W [N, K] in the activation dtype (bit-exact target).

    Composition of checkpoint.py:186-259 (unpack, restore, expand) and the
    activation-dtype cast of gptq_layer.py:568-569.
    """
    n = np.asarray(qweight).shape[1]
    k = np.asarray(qweight).shape[0] * 32 // bits
    q = unpack_int_weights(qweight, bits, (n, k))
    z = restore_zeros(unpack_zeros(qzeros, bits, n), bits, checkpoint_format)
    return round_to(dequant_fp32(q, scales, z, g_idx), dtype)


def to_f32(w, dtype: str) -> np.ndarray:
    if dtype in ("bf16", "bfloat16"):
        return bf16_bits_to_f32(w)
    return np.asarray(w).astype(np.float32)


def linear_ref(x, w, dtype="fp16", bias=None) -> np.ndarray:
    """fp32-accumulated reference of ``F.linear(x, W, bias)`` (gptq_layer.py:572).

    ``x`` and ``w`` are given in the activation dtype (bf16 as bit patterns);
    products and sums are formed in float64, the result returned in fp32.
    """
    xf = to_f32(x, dtype).astype(np.float64)
    wf = to_f32(w, dtype).astype(np.float64)
    y = xf @ wf.T
    if bias is not None:
        y = y + to_f32(bias, dtype).astype(np.float64)
    return y.astype(np.float32)


def gptq_forward(x, qweight, qzeros, scales, g_idx, bits, checkpoint_format="gptq",
                 dtype="fp16", bias=None) -> np.ndarray:
    """Whole HF-path forward (gptq_layer.py:515-574): dequant, cast, linear."""
    w = dequantize(qweight, qzeros, scales, g_idx, bits, checkpoint_format, dtype)
    return linear_ref(x, w, dtype, bias)
