"""Golden fixtures (tests/golden/*.npz): the oracle still reproduces them
(CPU), and the HIP path matches them (GPU)."""

import glob
import os

import numpy as np
import pytest

from oracle import dbf as od
from oracle import gptq as og

HERE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")
GPTQ = sorted(glob.glob(os.path.join(HERE, "gptq_*.npz")))


def _load(p):
    with np.load(p, allow_pickle=False) as f:
        return {k: f[k] for k in f.files}


@pytest.mark.parametrize("path", GPTQ, ids=os.path.basename)
def test_oracle_reproduces_gptq_golden(path):
    d = _load(path)
    bits = int(d["bits"])
    n, k = d["codes"].shape
    assert np.array_equal(og.unpack_int_weights(d["qweight"], bits, (n, k)), d["codes"])
    assert np.array_equal(og.restore_zeros(og.unpack_zeros(d["qzeros"], bits, n), bits), d["zeros"])
    w16 = og.dequantize(d["qweight"], d["qzeros"], d["scales"], d["g_idx"], bits, "gptq", "fp16")
    assert np.array_equal(w16.view(np.uint16), d["w16"])
    wbf = og.dequantize(d["qweight"], d["qzeros"], d["scales"], d["g_idx"], bits, "gptq", "bf16")
    assert np.array_equal(wbf, d["wbf16"])
    assert np.array_equal(og.linear_ref(d["x"], w16), d["y"])


def test_oracle_reproduces_dbf_golden():
    d = _load(os.path.join(HERE, "dbf_k96_n40.npz"))
    k, n, r = int(d["k"]), int(d["n"]), int(d["r"])
    assert np.array_equal(od.unpack_binary_factor(d["bp1"], (r, k)), d["S2"])
    assert np.array_equal(od.unpack_binary_factor(d["bp3"], (n, r)), d["S1"])
    y = od.dbf_forward(d["x"], d["s0"], d["bp1"], d["s2"], d["bp3"], d["s4"], k, r, n)
    assert np.array_equal(y, d["y"])


@pytest.mark.gpu
@pytest.mark.parametrize("path", GPTQ, ids=os.path.basename)
def test_hip_matches_gptq_golden(dev, path):
    import torch

    from onecompression_amd import ops

    d = _load(path)
    bits, gs = int(d["bits"]), int(d["group_size"])
    t = {k: torch.from_numpy(np.ascontiguousarray(d[k])).to(dev) for k in ("qweight", "qzeros", "scales", "g_idx", "x")}
    codes = ops.gptq_unpack_codes(t["qweight"], bits).cpu().numpy()
    assert np.array_equal(codes, d["codes"].astype(np.int32))
    w16 = ops.gptq_dequant(t["qweight"], t["qzeros"], t["scales"], t["g_idx"], bits, gs).cpu().numpy()
    assert np.array_equal(w16.view(np.uint16), d["w16"])
    wbf = ops.gptq_dequant(t["qweight"], t["qzeros"], t["scales"], t["g_idx"], bits, gs,
                           dtype=torch.bfloat16).view(torch.int16).cpu().numpy().view(np.uint16)
    assert np.array_equal(wbf, d["wbf16"])
    prep = ops.gptq_prepare(t["qweight"], t["qzeros"], t["scales"], t["g_idx"], bits, gs)
    y = ops.gptq_gemm(t["x"], prep).float().cpu().numpy()
    assert np.max(np.abs(y - d["y"])) / np.max(np.abs(d["y"])) <= 1e-2


@pytest.mark.gpu
def test_hip_matches_dbf_golden(dev):
    import torch

    from onecompression_amd import dbf_ops

    d = _load(os.path.join(HERE, "dbf_k96_n40.npz"))
    k, n, r = int(d["k"]), int(d["n"]), int(d["r"])
    t = {key: torch.from_numpy(np.ascontiguousarray(d[key])).to(dev) for key in ("bp1", "bp3", "s0", "s2", "s4", "x")}
    assert np.array_equal(dbf_ops.unpack_signs(t["bp1"], r, k).cpu().numpy(), d["S2"])
    prep = dbf_ops.dbf_prepare(t["s0"], t["bp1"], t["s2"], t["bp3"], t["s4"], k, r, n)
    y = dbf_ops.dbf_forward(t["x"], [prep]).float().cpu().numpy()
    assert np.max(np.abs(y - d["y"])) / np.max(np.abs(d["y"])) <= 1e-2
