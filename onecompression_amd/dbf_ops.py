"""Torch front end of the DBF / MDBF sign-matmul C ABI.

- :func:`dbf_prepare` / :func:`dbf_forward`: DBF parts
  (vllm_plugins/dbf/vllm_plugin.py:275-294, :330-381): per part
  ``t = s2 * (S2 @ (s0 * x))`` then ``y = s4 * (S1 @ t)``; fused parts write
  their column slice of one output (no ``torch.cat``) and bias is added once.
- :func:`mdbf_prepare_path` / :func:`mdbf_forward`: MDBF P-path layers
  (onecomp/quantizer/mdbf/mdbf_layer.py:307-344, :412-420):
  ``u_p = sum_k Q_V[:, k] * (S_B @ (B_amp[:, k] * x))`` then
  ``y = sum_{p,k} A_amp[:, k] * (S_A @ (Q_U[:, k] * u_p))``.
"""

from __future__ import annotations

import ctypes
from dataclasses import dataclass, field
from typing import Dict, List, Optional

import torch

from . import _native as N
from .ops import _DT, _need, _ptr, _stream


class OcSignTerm(ctypes.Structure):
    _fields_ = [("packed", ctypes.c_void_p), ("in_", ctypes.c_void_p), ("pre", ctypes.c_void_p),
                ("post", ctypes.c_void_p), ("Kd", ctypes.c_int), ("ld_in", ctypes.c_int)]


@dataclass
class SignFactor:
    """A +-1 factor (R x Kd) repacked into the kernel's sign layout."""

    packed: torch.Tensor
    R: int
    Kd: int
    unit_k: int


def sign_layout(R: int, Kd: int):
    nbytes, kpad, uk = ctypes.c_size_t(), ctypes.c_int(), ctypes.c_int()
    N.call("oc_dbf_layout", R, Kd, ctypes.byref(nbytes), ctypes.byref(kpad), ctypes.byref(uk))
    return nbytes.value, kpad.value, uk.value


def sign_prepare(bp: torch.Tensor, R: int, Kd: int) -> SignFactor:
    """Repack uint8 MSB-first flat signs (dbf_layer.py:32-44 layout)."""
    _need(bp, "bp", torch.uint8, align=1)
    if bp.numel() < (R * Kd + 7) // 8:
        raise ValueError(f"sign buffer has {bp.numel()} bytes, {R}x{Kd} needs {(R * Kd + 7) // 8}")
    nbytes, _kp, uk = sign_layout(R, Kd)
    packed = torch.empty(nbytes, dtype=torch.uint8, device=bp.device)
    N.call("oc_dbf_prepare", _ptr(bp), R, Kd, _ptr(packed), _stream(bp.device))
    return SignFactor(packed, R, Kd, uk)


def unpack_signs(bp: torch.Tensor, R: int, Kd: int) -> torch.Tensor:
    """int8 +-1 [R, Kd] (replaces unpack_sign_bits, vllm_plugins/dbf/modules/naive.py:9-42)."""
    _need(bp, "bp", torch.uint8, align=1)
    out = torch.empty((R, Kd), dtype=torch.int8, device=bp.device)
    N.call("oc_dbf_unpack_signs", _ptr(bp), R, Kd, _ptr(out), _stream(bp.device))
    return out


def _vec(t: Optional[torch.Tensor], dtype: torch.dtype, n: int, cache: Dict, key) -> Optional[torch.Tensor]:
    """A scale vector in the activation dtype, zero-padded to a multiple of 8 (cached).

    The kernel reads pre scales in 8-element chunks; the zero tail keeps the
    padded k positions finite (their activations are zero too).
    """
    if t is None:
        return None
    k = (key, dtype)
    v = cache.get(k)
    if v is None:
        if _capturing(t):
            raise RuntimeError(f"scale vector {key} built under HIP graph capture (it would live in the "
                               "graph's private pool); prepare the layer with dbf_prepare/mdbf_prepare_path")
        src = t.reshape(-1)
        if src.numel() != n:
            raise ValueError(f"scale vector {key} has {src.numel()} entries, expected {n}")
        v = torch.zeros(_ld(n), dtype=dtype, device=src.device)
        v[:n].copy_(src)
        cache[k] = v
    return v


def _capturing(t: torch.Tensor) -> bool:
    return t.is_cuda and torch.cuda.is_current_stream_capturing()


def _fill_vecs(cache: Dict, items) -> None:
    """Build a layer's cached scale vectors for both activation dtypes at prepare time, so that no
    forward call creates them: one created during HIP graph capture would live in the graph's
    private memory pool (and the capture would re-run its fill on every replay)."""
    for dt in _DT:
        for t, n, key in items:
            _vec(t, dt, n, cache, key)


def sign_gemm(terms, M: int, R: int, dtype: torch.dtype, out: torch.Tensor, ld_out: int,
              fill_to: int = 0, bias: Optional[torch.Tensor] = None) -> None:
    """Launch oc_sign_gemm; ``terms`` = list of (SignFactor, in [M, ld_in], pre, post)."""
    if not 1 <= len(terms) <= 4:
        raise NotImplementedError(f"{len(terms)} sign terms in one output; at most 4 are supported")
    arr = _terms_array(terms, dtype)
    nbytes = N.load().oc_sign_workspace_bytes(arr, len(terms), M, R)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=out.device) if nbytes else None
    N.call("oc_sign_gemm", arr, len(terms), M, R, _DT[dtype], _ptr(bias), _ptr(out), ld_out,
           fill_to, _ptr(ws), nbytes, _stream(out.device))


def _terms_array(terms, dtype):
    arr = (OcSignTerm * len(terms))()
    for i, (f, x, pre, post) in enumerate(terms):
        if x.dtype != dtype:
            raise TypeError("all terms must use the activation dtype")
        if x.stride(-1) != 1 or x.data_ptr() % 16 or x.stride(0) % 8:
            raise ValueError("term input rows must be contiguous, 16-byte aligned, stride % 8 == 0")
        arr[i] = OcSignTerm(f.packed.data_ptr(), x.data_ptr(), 0 if pre is None else pre.data_ptr(),
                            0 if post is None else post.data_ptr(), f.Kd, x.stride(0))
    return arr


def sign_gemm_batch(problems, M: int, R: int, dtype: torch.dtype, outs: List[torch.Tensor], ld_out: int,
                    fill_to: int = 0) -> None:
    """Launch oc_sign_gemm_batch: independent single-term problems (SignFactor, in, pre, post), problem p
    into outs[p] (each [M, ld_out]); one launch where the problems share a unit size and pre presence."""
    if not 1 <= len(problems) <= 4 or len(outs) != len(problems):
        raise NotImplementedError(f"{len(problems)} problems in one batch; 1 to 4 with one output each")
    arr = _terms_array(problems, dtype)
    ptrs = (ctypes.c_void_p * len(outs))(*[o.data_ptr() for o in outs])
    nbytes = N.load().oc_sign_batch_workspace_bytes(arr, len(problems), M, R)
    ws = torch.empty(nbytes, dtype=torch.uint8, device=outs[0].device) if nbytes else None
    N.call("oc_sign_gemm_batch", arr, len(problems), M, R, _DT[dtype], ptrs, ld_out, fill_to, _ptr(ws), nbytes,
           _stream(outs[0].device))


def _ld(n: int) -> int:
    return (n + 7) // 8 * 8


# ---------------------------------------------------------------------------------- DBF

@dataclass
class DBFPart:
    s0: torch.Tensor
    s2: torch.Tensor
    s4: torch.Tensor
    S2: SignFactor  # r x K  (bp1)
    S1: SignFactor  # N x r  (bp3)
    in_features: int
    mid: int
    out_features: int
    _cache: Dict = field(default_factory=dict, repr=False)


def dbf_prepare(s0, bp1, s2, bp3, s4, in_features: int, mid: int, out_features: int) -> DBFPart:
    """One DBF part: scaling0 [K], bp1 (r x K), scaling2 [r], bp3 (N x r), scaling4 [N]."""
    S2 = sign_prepare(bp1, mid, in_features)
    S1 = sign_prepare(bp3, out_features, mid)
    p = DBFPart(s0, s2, s4, S2, S1, in_features, mid, out_features)
    _fill_vecs(p._cache, [(s0, in_features, "s0"), (s2, mid, "s2"), (s4, out_features, "s4")])
    return p


def dbf_forward(x: torch.Tensor, parts: List[DBFPart], bias: Optional[torch.Tensor] = None,
                out: Optional[torch.Tensor] = None) -> torch.Tensor:
    if x.dtype not in _DT:
        raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
    k = parts[0].in_features
    lead = x.shape[:-1]
    x2 = x.reshape(-1, k)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    m = x2.shape[0]
    dev, dt = x2.device, x2.dtype
    n_total = sum(p.out_features for p in parts)
    if out is None:
        out = torch.empty((m, n_total), dtype=dt, device=dev)
    off = 0
    for i, p in enumerate(parts):
        c = p._cache
        t = torch.empty((m, _ld(p.mid)), dtype=dt, device=dev)
        sign_gemm([(p.S2, x2, _vec(p.s0, dt, k, c, "s0"), _vec(p.s2, dt, p.mid, c, "s2"))], m, p.mid,
                  dt, t, t.stride(0), fill_to=t.stride(0))
        b = None if bias is None else bias.reshape(-1)[off:off + p.out_features].to(dt).contiguous()
        sign_gemm([(p.S1, t, None, _vec(p.s4, dt, p.out_features, c, "s4"))], m, p.out_features, dt,
                  out[:, off:], n_total, bias=b)
        off += p.out_features
    return out.reshape(*lead, n_total)


# ---------------------------------------------------------------------------------- MDBF

@dataclass
class MDBFPath:
    A: SignFactor  # n x r
    B: SignFactor  # r x m
    A_amp: torch.Tensor  # [l, n] (transposed for contiguous columns)
    B_amp: torch.Tensor  # [l, m]
    Q_U: torch.Tensor    # [l, r]
    Q_V: torch.Tensor    # [l, r]
    n: int
    r: int
    m: int
    l: int
    _cache: Dict = field(default_factory=dict, repr=False)


def mdbf_prepare_path(a_packed, a_shape, b_packed, b_shape, a_amp, b_amp, qu_amp, qv_amp) -> MDBFPath:
    """One MDBF path (mdbf_layer.py:516-610 keys: A/B_sign_packed, A/B/Q_U/Q_V_amp)."""
    n, r = int(a_shape[0]), int(a_shape[1])
    r2, m = int(b_shape[0]), int(b_shape[1])
    if r != r2:
        raise ValueError(f"A is {n}x{r} but B is {r2}x{m}")
    l = a_amp.reshape(n, -1).shape[1]
    A = sign_prepare(a_packed, n, r)
    B = sign_prepare(b_packed, r, m)

    def tr(t, d):
        return t.reshape(d, l).t().contiguous()

    p = MDBFPath(A, B, tr(a_amp, n), tr(b_amp, m), tr(qu_amp, r), tr(qv_amp, r), n, r, m, l)
    _fill_vecs(p._cache, [v for k in range(l) for v in ((p.B_amp[k], m, f"b{k}"), (p.Q_V[k], r, f"qv{k}"),
                                                          (p.Q_U[k], r, f"qu{k}"), (p.A_amp[k], n, f"a{k}"))])
    return p


def mdbf_forward(x: torch.Tensor, paths: List[MDBFPath], bias: Optional[torch.Tensor] = None) -> torch.Tensor:
    if x.dtype not in _DT:
        raise TypeError(f"activations must be fp16 or bf16, got {x.dtype}")
    mdim, ndim = paths[0].m, paths[0].n
    lead = x.shape[:-1]
    x2 = x.reshape(-1, mdim)
    if not x2.is_contiguous() or x2.data_ptr() % 16:
        x2 = x2.contiguous()
    rows = x2.shape[0]
    dev, dt = x2.device, x2.dtype
    stage2 = []
    us = [torch.empty((rows, _ld(p.r)), dtype=dt, device=dev) for p in paths]
    rank = [[(p.B, x2, _vec(p.B_amp[k], dt, mdim, p._cache, f"b{k}"), _vec(p.Q_V[k], dt, p.r, p._cache, f"qv{k}"))
             for k in range(p.l)] for p in paths]
    if len(paths) > 1 and all(p.l == 1 and p.r == paths[0].r for p in paths):
        # the paths' rank stages are independent problems on the same x: one batched launch
        r0 = paths[0].r
        sign_gemm_batch([t[0] for t in rank], rows, r0, dt, us, us[0].stride(0), fill_to=us[0].stride(0))
    else:
        for p, terms, u in zip(paths, rank, us):
            sign_gemm(terms, rows, p.r, dt, u, u.stride(0), fill_to=u.stride(0))
    for p, u in zip(paths, us):
        c = p._cache
        stage2 += [(p.A, u, _vec(p.Q_U[k], dt, p.r, c, f"qu{k}"), _vec(p.A_amp[k], dt, ndim, c, f"a{k}"))
                   for k in range(p.l)]
    y = torch.empty((rows, ndim), dtype=dt, device=dev)
    b = None if bias is None else bias.reshape(-1).to(dt).contiguous()
    sign_gemm(stage2, rows, ndim, dt, y, ndim, bias=b)
    return y.reshape(*lead, ndim)
