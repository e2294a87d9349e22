"""HF-path drop-ins (GPTQLinear, DoubleBinaryLinear, MultipathMDBFLinear): construction and
state-dict behaviour on CPU; forward parity against the oracle on the GPU."""

import numpy as np
import pytest
import torch

from oracle import dbf as od
from oracle import gptq as og
from onecompression_amd import hf, synth


def _gptq_sd(bits=4, k=256, n=64, gs=32, seed=0, fmt="gptq"):
    c = synth.gptq_case("t", k, n, bits, gs, False, seed)
    return c, {"qweight": c.qweight, "scales": c.scales, "qzeros": c.qzeros,
               "g_idx": torch.from_numpy(og.default_g_idx(k, gs))}


def test_gptq_from_saved_state_empty_then_load():
    c, sd = _gptq_sd()
    layer = hf.GPTQLinear.from_saved_state(sd, 256, 64, 4, 32, empty=True)
    assert set(layer.state_dict()) == {"qweight", "scales", "qzeros", "g_idx"}
    assert all(torch.count_nonzero(v) == 0 for v in layer.state_dict().values())
    layer.load_state_dict(sd)
    assert torch.equal(layer.qweight, c.qweight)


def test_gptq_default_g_idx_and_wbits_normalisation():
    _, sd = _gptq_sd()
    del sd["g_idx"]
    layer = hf.GPTQLinear.from_saved_state(sd, 256, 64, 4.0, 32)
    assert layer.wbits == 4 and type(layer.wbits) is int
    assert torch.equal(layer.g_idx, torch.arange(256, dtype=torch.int32) // 32)
    layer = hf.GPTQLinear.from_saved_state(sd, 256, 64, 4, -1)
    assert torch.count_nonzero(layer.g_idx) == 0
    for bad in (2.5, True):
        with pytest.raises(ValueError):
            hf.GPTQLinear.from_saved_state(sd, 256, 64, bad, 32)


def test_layers_refuse_cpu_tensors():
    _, sd = _gptq_sd()
    layer = hf.GPTQLinear.from_saved_state(sd, 256, 64, 4, 32)
    with pytest.raises(RuntimeError, match="HIP device"):
        layer(torch.zeros(1, 256, dtype=torch.float16))


def _dbf_sd(k, n, seed, bias=False):
    rng = np.random.default_rng(seed)
    r = od.mid_features(1.0, k, n)
    sd = {"scaling0": (np.abs(rng.normal(0, 0.05, k)) + 1e-3).astype(np.float16),
          "scaling2": (np.abs(rng.normal(0, 0.05, r)) + 1e-3).astype(np.float16),
          "scaling4": (np.abs(rng.normal(0, 0.05, n)) + 1e-3).astype(np.float16),
          "bp1": od.pack_binary(rng.choice([-1, 1], size=(r, k))),
          "bp3": od.pack_binary(rng.choice([-1, 1], size=(n, r)))}
    if bias:
        sd["bias"] = rng.normal(0, 0.01, n).astype(np.float16)
    return r, {k_: torch.from_numpy(np.ascontiguousarray(v)) for k_, v in sd.items()}


def test_dbf_from_saved_state_keys():
    r, sd = _dbf_sd(128, 96, 1, bias=True)
    layer = hf.DoubleBinaryLinear.from_saved_state(sd, 128, 96, empty=True, target_bits=1.0)
    assert set(layer.state_dict()) == set(sd)
    assert layer._bp1_shape == (r, 128) and layer._bp3_shape == (96, r)
    layer.load_state_dict(sd)
    assert torch.equal(layer.bp3, sd["bp3"])


def _mdbf_sd(n, m, P, l, seed, bias=False):
    rng = np.random.default_rng(seed)
    r = od.mid_features(1.0, m, n)
    sd, paths = {}, []
    for p in range(P):
        amp = lambda *s: (np.abs(rng.normal(0, 0.3, s)) + 1e-2).astype(np.float16)  # noqa: E731
        d = dict(A_sign_packed=od.pack_binary(rng.choice([-1, 1], size=(n, r))), A_shape=(n, r),
                 B_sign_packed=od.pack_binary(rng.choice([-1, 1], size=(r, m))), B_shape=(r, m),
                 A_amp=amp(n, l), B_amp=amp(m, l), Q_U_amp=amp(r, l), Q_V_amp=amp(r, l))
        paths.append(d)
        for k_ in ("A_sign_packed", "B_sign_packed", "A_amp", "B_amp", "Q_U_amp", "Q_V_amp"):
            sd[f"paths.{p}.{k_}"] = torch.from_numpy(np.ascontiguousarray(d[k_]))
        sd[f"paths.{p}._A_sign_shape"] = torch.tensor([n, r])
        sd[f"paths.{p}._B_sign_shape"] = torch.tensor([r, m])
    if bias:
        sd["bias"] = torch.from_numpy(rng.normal(0, 0.01, n).astype(np.float16))
    return paths, sd


def test_mdbf_from_saved_state_and_validation():
    _, sd = _mdbf_sd(96, 64, 2, 2, 3, bias=True)
    layer = hf.MultipathMDBFLinear.from_saved_state(sd, 64, 96, empty=True)
    assert layer.P == 2 and layer.paths[0].l == 2
    assert set(layer.state_dict()) == set(sd)
    layer.load_state_dict(sd)
    hf.MultipathMDBFLinear.validate_saved_state(sd, layer_name="x", expected_paths=2, expects_bias=True)
    with pytest.raises(ValueError, match="path indices"):
        hf.MultipathMDBFLinear.validate_saved_state(sd, layer_name="x", expected_paths=3, expects_bias=True)
    with pytest.raises(ValueError, match="bias mismatch"):
        hf.MultipathMDBFLinear.validate_saved_state(sd, layer_name="x", expected_paths=2, expects_bias=False)
    with pytest.raises(ValueError, match="no `paths"):
        hf.MultipathMDBFLinear.from_saved_state({"bias": sd["bias"]}, 64, 96)


# ------------------------------------------------------------------------------------ GPU


def _rel(y, ref):
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.gpu
@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("fmt", ["gptq", "gptq_v2"])
def test_gptq_linear_forward(dev, bits, fmt):
    """gptq_layer.py:515-574 via from_saved_state, both checkpoint formats, group 32."""
    c, sd = _gptq_sd(bits, 256, 96 if bits != 3 else 64, 32, seed=bits, fmt=fmt)
    layer = hf.GPTQLinear.from_saved_state({k: v.to(dev) for k, v in sd.items()}, 256, c.out_features, bits, 32,
                                           checkpoint_format=fmt)
    x = synth.activations(3, 256, seed=2)
    y = layer(x.to(dev)).float().cpu().numpy()
    w = og.dequantize(c.qweight.numpy(), c.qzeros.numpy(), c.scales.numpy(), og.default_g_idx(256, 32), bits,
                      fmt, "fp16")
    assert _rel(y, og.linear_ref(x.numpy(), w, "fp16")) <= 1e-2


@pytest.mark.gpu
def test_gptq_linear_replace_then_load_and_reload(dev):
    """empty=True, then load_state_dict (the HF loader's flow); a second load re-prepares."""
    c1, sd1 = _gptq_sd(4, 512, 128, 128, seed=11)
    c2, sd2 = _gptq_sd(4, 512, 128, 128, seed=12)
    sd1["bias"] = (torch.randn(128) * 0.05).half()
    sd2["bias"] = (torch.randn(128) * 0.05).half()
    layer = hf.GPTQLinear.from_saved_state(sd1, 512, 128, 4, 128, empty=True).to(dev)
    x = synth.activations(5, 512, seed=3)
    for c, sd in ((c1, sd1), (c2, sd2)):
        layer.load_state_dict(sd)
        y = layer(x.to(dev)).float().cpu().numpy()
        w = og.dequantize(c.qweight.numpy(), c.qzeros.numpy(), c.scales.numpy(), og.default_g_idx(512, 128), 4,
                          "gptq", "fp16")
        ref = og.linear_ref(x.numpy(), w, "fp16", sd["bias"].numpy())
        assert _rel(y, ref) <= 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("m", [1, 9, 140])
def test_double_binary_linear_forward(dev, m):
    k, n = 256, 192
    r, sd = _dbf_sd(k, n, 5, bias=True)
    layer = hf.DoubleBinaryLinear.from_saved_state(sd, k, n, empty=True).to(dev)
    layer.load_state_dict(sd)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half()
    y = layer(x.to(dev)).float().cpu().numpy()
    s = {k_: v.numpy() for k_, v in sd.items()}
    ref = od.dbf_forward(x.numpy(), s["scaling0"], s["bp1"], s["scaling2"], s["bp3"], s["scaling4"], k, r, n)
    assert _rel(y, ref + s["bias"].astype(np.float32)) <= 1e-2


@pytest.mark.gpu
@pytest.mark.parametrize("P,l,m_rows", [(2, 1, 3), (2, 2, 1), (1, 2, 130)])
def test_multipath_mdbf_linear_forward(dev, P, l, m_rows):
    n, m = 192, 128
    paths, sd = _mdbf_sd(n, m, P, l, 7, bias=True)
    layer = hf.MultipathMDBFLinear.from_saved_state(sd, m, n, empty=True).to(dev)
    layer.load_state_dict(sd)
    x = torch.randn(m_rows, m, generator=torch.Generator().manual_seed(4)).half()
    y = layer(x.to(dev)).float().cpu().numpy()
    ref = od.mdbf_forward(x.numpy(), paths) + sd["bias"].numpy().astype(np.float32)
    assert _rel(y, ref) <= 1e-2
