"""HF-path drop-ins: quantized ``nn.Module`` layers backed by the HIP kernels.

OneComp's HF loader (onecomp/quantized_model_loader.py:1044-1089) replaces
each ``nn.Linear`` with a module built by ``from_saved_state(..., empty=True)``
and then fills its buffers with ``load_state_dict``.  These classes keep those
constructors, attribute names and state-dict keys:

- :class:`GPTQLinear` (onecomp/quantizer/gptq/gptq_layer.py:247-714):
  ``qweight`` / ``scales`` / ``qzeros`` / ``g_idx`` (/ ``perm``, ``bias``);
  forward = F.linear(x, RNE(s * (q - z)), bias) (gptq_layer.py:515-574).
- :class:`DoubleBinaryLinear` (onecomp/quantizer/dbf/dbf_layer.py:121-355):
  ``scaling0/2/4`` parameters, ``bp1`` / ``bp3`` buffers, ``bias``; the
  five-stage forward of dbf_layer.py:251-268.
- :class:`MultipathMDBFLinear` (onecomp/quantizer/mdbf/mdbf_layer.py:370-610):
  ``paths.{p}.{A,B}_sign_packed``, ``paths.{p}.{A,B,Q_U,Q_V}_amp``, ``bias``;
  forward = sum of the paths (mdbf_layer.py:412-420), each path the staged
  form of mdbf_layer.py:307-336.

Weights are repacked into the kernel layouts on the first forward after the
buffers change (tracked through the tensors' version counters and data
pointers), so the "replace, then load_state_dict" flow works unchanged.  The
layers run on a HIP device only; on CPU tensors they raise (no fallback).
Out of scope: the constructors that take in-process quantization results
(quantization itself is not part of this build) and GemLite.
"""

from __future__ import annotations

from typing import Dict, List, Mapping, Optional

import torch
from torch import nn

from . import _native as N
from . import dbf_ops, ops


def _normalize_wbits(wbits) -> int:
    """wbits as a builtin int.  Integers (bool excluded) and integral floats are accepted; any other
    value raises ValueError (the contract of gptq_layer.py:214-227)."""
    integral = (isinstance(wbits, int) and not isinstance(wbits, bool)) or \
        (isinstance(wbits, float) and wbits.is_integer())
    if not integral:
        raise ValueError(f"wbits must be an integer value, got {wbits!r}.")
    return int(wbits)


def _stamp(tensors) -> tuple:
    return tuple((t.data_ptr(), t._version, str(t.device)) for t in tensors if t is not None)


def _need_device(x: torch.Tensor, name: str) -> None:
    if x.device.type != "cuda":
        raise RuntimeError(f"{name} (onecomp-amd) runs on a HIP device; got a {x.device} tensor")


class GPTQLinear(nn.Module):
    """GPTQ layer in the AutoGPTQ checkpoint layout, served by ``oc_gptq_gemm``."""

    @classmethod
    def from_saved_state(cls, layer_state_dict: Mapping[str, torch.Tensor], in_features: int,
                         out_features: int, wbits, groupsize: int = -1, actorder: bool = False,
                         empty: bool = False, checkpoint_format: str = "gptq") -> "GPTQLinear":
        """gptq_layer.py:630-714: buffers from a layer state dict (zeros when ``empty``)."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.in_features, self.out_features = in_features, out_features
        self.wbits, self.groupsize, self.actorder = _normalize_wbits(wbits), groupsize, actorder
        self.checkpoint_format = checkpoint_format
        self._weight_is_packed = self.wbits != 1  # 1-bit checkpoints are stored unpacked
        self.using_gemlite = False
        self._prep = None
        self._prep_stamp = None

        missing = [k for k in ("qweight", "scales", "qzeros") if k not in layer_state_dict]
        if missing:
            raise KeyError(f"GPTQ layer state is missing {missing}")
        take = {k: layer_state_dict[k] for k in ("qweight", "scales", "qzeros", "g_idx", "perm", "bias")
                if layer_state_dict.get(k) is not None}
        if empty:  # "replace, then load_state_dict": same shapes and dtypes, zero contents
            take = {k: torch.zeros_like(t) for k, t in take.items()}
        if "g_idx" not in take:  # no act-order tensor saved: the sequential groups k // groupsize
            k = torch.arange(in_features, dtype=torch.int32, device=take["qweight"].device)
            take["g_idx"] = k // groupsize if groupsize != -1 else torch.zeros_like(k)
        for key in ("qweight", "scales", "qzeros", "g_idx", "perm", "bias"):
            if key in take:
                self.register_buffer(key, take[key])
            else:
                setattr(self, key, None)
        return self

    def _prepared(self) -> ops.PreparedGPTQ:
        if self.wbits not in (2, 3, 4, 8):
            raise NotImplementedError(f"GPTQLinear with wbits={self.wbits}: the kernels take 2/3/4/8 bits")
        stamp = _stamp([self.qweight, self.qzeros, self.scales, self.g_idx])
        if self._prep is None or stamp != self._prep_stamp:
            gs = self.groupsize if self.groupsize and self.groupsize > 0 else -1
            fmt = N.OC_ZERO_V2 if self.checkpoint_format == "gptq_v2" else N.OC_ZERO_V1
            g_idx = self.g_idx.to(torch.int32).contiguous()
            self._prep = ops.gptq_prepare(self.qweight.contiguous(), self.qzeros.contiguous(),
                                          self.scales.to(torch.float16).contiguous(), g_idx, self.wbits,
                                          gs if gs > 0 else self.in_features, fmt)
            self._prep_stamp = stamp
        return self._prep

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _need_device(x, "GPTQLinear")
        prep = self._prepared()
        bias = None if self.bias is None else self.bias.to(x.dtype)
        return ops.gptq_gemm(x, prep, bias)

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, wbits={self.wbits}, "
                f"groupsize={self.groupsize}, actorder={self.actorder}")


class DoubleBinaryLinear(nn.Module):
    """DBF layer W ~ diag(s4) S1 diag(s2) S2 diag(s0), served by ``oc_sign_gemm``."""

    @classmethod
    def from_saved_state(cls, layer_state_dict: Mapping[str, torch.Tensor], in_features: int,
                         out_features: int, empty: bool = False,
                         target_bits: Optional[float] = None) -> "DoubleBinaryLinear":
        """dbf_layer.py:303-355."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.target_bits = target_bits
        self.in_features, self.out_features = in_features, out_features

        def _p(k):
            t = layer_state_dict[k]
            return torch.zeros_like(t) if empty else t

        self.scaling0 = nn.Parameter(_p("scaling0"), requires_grad=False)
        self.scaling2 = nn.Parameter(_p("scaling2"), requires_grad=False)
        self.scaling4 = nn.Parameter(_p("scaling4"), requires_grad=False)
        mid = layer_state_dict["scaling2"].numel()
        self._bp1_shape = (mid, in_features)
        self._bp3_shape = (out_features, mid)
        self.register_buffer("bp1", _p("bp1"))
        self.register_buffer("bp3", _p("bp3"))
        bias = layer_state_dict.get("bias")
        if bias is not None:
            self.register_buffer("bias", torch.zeros_like(bias) if empty else bias)
        else:
            self.bias = None
        self.use_gemlite = False
        self._part = None
        self._part_stamp = None
        return self

    def _prepared(self) -> dbf_ops.DBFPart:
        stamp = _stamp([self.bp1, self.bp3, self.scaling0, self.scaling2, self.scaling4])
        if self._part is None or stamp != self._part_stamp:
            mid = self._bp1_shape[0]
            self._part = dbf_ops.dbf_prepare(self.scaling0.data.reshape(-1), self.bp1.contiguous(),
                                             self.scaling2.data.reshape(-1), self.bp3.contiguous(),
                                             self.scaling4.data.reshape(-1), self.in_features, mid,
                                             self.out_features)
            self._part_stamp = stamp
        return self._part

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _need_device(x, "DoubleBinaryLinear")
        bias = None if self.bias is None else self.bias.to(x.dtype)
        return dbf_ops.dbf_forward(x, [self._prepared()], bias)


def mdbf_path_indices(layer_state_dict: Mapping[str, torch.Tensor]) -> set:
    """Path indices present as ``paths.{p}.*`` keys (mdbf_layer.py:46-60)."""
    out = set()
    for key in layer_state_dict:
        parts = key.split(".")
        if parts[0] == "paths" and len(parts) >= 2 and parts[1].isdigit():
            out.add(int(parts[1]))
    return out


class MDBFLinear(nn.Module):
    """One MDBF path (buffers of mdbf_layer.py:111-163 / :581-590)."""

    def __init__(self, n: int, r: int, m: int, tensors: Dict[str, torch.Tensor]):
        super().__init__()
        self.n, self.r, self.m = n, r, m
        self.register_buffer("A_sign_packed", tensors["A_sign_packed"])
        self.register_buffer("B_sign_packed", tensors["B_sign_packed"])
        dev = tensors["A_amp"].device
        self.register_buffer("_A_sign_shape", torch.tensor([n, r], dtype=torch.int64, device=dev))
        self.register_buffer("_B_sign_shape", torch.tensor([r, m], dtype=torch.int64, device=dev))
        for k in ("A_amp", "B_amp", "Q_U_amp", "Q_V_amp"):
            self.register_buffer(k, tensors[k])
        self.l = self.A_amp.shape[1]
        self.use_gemlite = False
        self._path = None
        self._path_stamp = None

    def _prepared(self) -> dbf_ops.MDBFPath:
        stamp = _stamp([self.A_sign_packed, self.B_sign_packed, self.A_amp, self.B_amp, self.Q_U_amp,
                        self.Q_V_amp])
        if self._path is None or stamp != self._path_stamp:
            self._path = dbf_ops.mdbf_prepare_path(self.A_sign_packed.contiguous(), (self.n, self.r),
                                                   self.B_sign_packed.contiguous(), (self.r, self.m),
                                                   self.A_amp, self.B_amp, self.Q_U_amp, self.Q_V_amp)
            self._path_stamp = stamp
        return self._path

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _need_device(x, "MDBFLinear")
        return dbf_ops.mdbf_forward(x, [self._prepared()])


class MultipathMDBFLinear(nn.Module):
    """P-path MDBF layer, all paths summed inside one stage-2 launch."""

    @staticmethod
    def validate_saved_state(layer_state_dict: Mapping[str, torch.Tensor], *, layer_name: str,
                             expected_paths: Optional[int], expects_bias: bool) -> None:
        """mdbf_layer.py:462-515: a lost path or bias fails instead of loading a smaller layer."""
        idx = mdbf_path_indices(layer_state_dict)
        if expected_paths is not None and (len(idx) != expected_paths or (idx and max(idx) >= expected_paths)):
            raise ValueError(f"Incomplete MDBF checkpoint for {layer_name}: config records "
                             f"P={expected_paths} but the checkpoint has path indices {sorted(idx)}.")
        if ("bias" in layer_state_dict) != expects_bias:
            expected, found = ("a bias", "none") if expects_bias else ("no bias", "one")
            raise ValueError(f"MDBF checkpoint bias mismatch for {layer_name}: the model's nn.Linear "
                             f"expects {expected} but the checkpoint has {found}.")

    @classmethod
    def from_saved_state(cls, layer_state_dict: Mapping[str, torch.Tensor], in_features: int,
                         out_features: int, empty: bool = False,
                         target_bits: Optional[float] = None) -> "MultipathMDBFLinear":
        """mdbf_layer.py:516-610: P from the ``paths.{p}`` keys, l from A_amp's columns."""
        self = cls.__new__(cls)
        nn.Module.__init__(self)
        self.target_bits = target_bits
        self.n, self.m = out_features, in_features
        self.in_features, self.out_features = in_features, out_features

        def _t(k):
            t = layer_state_dict[k]
            return torch.zeros_like(t) if empty else t

        idx = mdbf_path_indices(layer_state_dict)
        if not idx:
            raise ValueError("MultipathMDBFLinear.from_saved_state: no `paths.{p}.*` keys found in "
                             "layer_state_dict.")
        self.P = max(idx) + 1
        paths: List[MDBFLinear] = []
        for p in range(self.P):
            pre = f"paths.{p}."
            r = layer_state_dict[f"{pre}Q_U_amp"].shape[0]
            paths.append(MDBFLinear(out_features, r, in_features,
                                    {k: _t(pre + k) for k in ("A_sign_packed", "B_sign_packed", "A_amp", "B_amp",
                                                              "Q_U_amp", "Q_V_amp")}))
        self.paths = nn.ModuleList(paths)
        bias = layer_state_dict.get("bias")
        if bias is not None:
            self.register_buffer("bias", torch.zeros_like(bias) if empty else bias)
        else:
            self.bias = None
        return self

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        _need_device(x, "MultipathMDBFLinear")
        bias = None if self.bias is None else self.bias.to(x.dtype)
        return dbf_ops.mdbf_forward(x, [p._prepared() for p in self.paths], bias)
