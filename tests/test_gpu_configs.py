"""Oracle parity at every BASELINE config and M, at the configs' full shapes (through the C ABI).

Configs 0-2 and 4 compare whole outputs with the float64 oracle (gptq_layer.py:515-574: bit-exact
dequantisation, then F.linear); config 4 at M = 4096 and 8192 compares one row of every 256-row
block over all columns and every row over a column sample (so every output tile, whole or cut
along K, is checked).  Config 3 compares DBF (dbf_layer.py:251-268) and MDBF P = 2
(mdbf_layer.py:412-420) at both MLP shapes.  Each test also holds a regression bound well below
the 1e-2 contract (measured errors are ~3e-4 in fp16 and ~2e-3 in bf16 outputs).
"""

import re

import numpy as np
import pytest
import torch

from oracle import dbf as od
from oracle import gptq as og
from onecompression_amd import _native as N
from onecompression_amd import dbf_ops, ops, synth

pytestmark = pytest.mark.gpu

BAR = 1e-2
TIGHT = {"fp16": 2e-3, "bf16": 6e-3}

_W = {}      # oracle dequantisation per (config, projection, dtype)
_PREP = {}   # repacked device layers per (config, projection)


def _np(t):
    return t.detach().cpu().numpy()


def _rel(y, ref):
    return float(np.max(np.abs(y - ref)) / max(float(np.max(np.abs(ref))), 1e-30))


def _bits16(t):
    return _np(t.cpu().view(torch.int16)).view(np.uint16)


def _case(cfg, idx):
    return synth.config_cases(cfg)[idx]


def _oracle_w(cfg, idx, dtype):
    key = (cfg, idx, dtype)
    if key not in _W:
        c = _case(cfg, idx)
        g = _np(c.g_idx) if c.g_idx is not None else og.default_g_idx(c.in_features, c.group_size)
        _W[key] = og.dequantize(_np(c.qweight), _np(c.qzeros), _np(c.scales), g, c.bits, "gptq", dtype)
    return _W[key]


def _prep(dev, cfg, idx):
    key = (cfg, idx)
    if key not in _PREP:
        c = _case(cfg, idx).to(dev)
        _PREP[key] = ops.gptq_prepare(c.qweight, c.qzeros, c.scales, c.g_idx, c.bits, c.group_size)
    return _PREP[key]


def _check(got, ref, dtype, what):
    r = _rel(got, ref)
    print(f"{what}: max rel err {r:.2e}")
    assert r <= BAR, f"{what}: {r:.3e} > {BAR}"
    assert r <= TIGHT[dtype], f"{what}: {r:.3e} above the regression bound {TIGHT[dtype]}"
    return r


def _run(dev, cfg, idx, m, dtype, seed):
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    x = synth.activations(m, _case(cfg, idx).in_features, td, seed=seed)
    y = ops.gptq_gemm(x.to(dev), _prep(dev, cfg, idx))
    torch.cuda.synchronize()
    return x, y


def _xin(x, dtype):
    return _bits16(x) if dtype == "bf16" else _np(x)


# ------------------------------------------------------------------------------ configs 0-2


@pytest.mark.parametrize("m", [1, 16])
def test_config0(dev, m):
    x, y = _run(dev, 0, 0, m, "fp16", seed=1000 + m)
    _check(_np(y.float()), og.linear_ref(_np(x), _oracle_w(0, 0, "fp16"), "fp16"), "fp16", f"cfg0 M={m}")


@pytest.mark.parametrize("m", [1, 8, 32, 128])
@pytest.mark.parametrize("idx", range(7))
def test_config1_projection(dev, idx, m):
    """The seven projections as separate linears (the reference's dispatch)."""
    x, y = _run(dev, 1, idx, m, "fp16", seed=1100 + 10 * idx + m)
    name = synth.CONFIG1[idx][0]
    _check(_np(y.float()), og.linear_ref(_np(x), _oracle_w(1, idx, "fp16"), "fp16"), "fp16", f"cfg1 {name} M={m}")


@pytest.mark.parametrize("m", [1, 8, 32, 128])
def test_config1_layer_calls(dev, m):
    """The four apply() calls of the bench step: qkv_proj as one fused module (q 4-bit | k, v
    8-bit, one grouped launch), o_proj, merged gate|up, down_proj."""
    names = [n for n, *_ in synth.CONFIG1]
    w = {n: _oracle_w(1, i, "fp16") for i, n in enumerate(names)}
    cases = {c.name: c for c in synth.config_cases(1)}
    x = synth.activations(m, 4096, torch.float16, seed=1200 + m)
    xd = x.to(dev)
    calls = synth.layer_calls(1)
    # qkv: q alone, k|v merged, served by oc_gptq_gemm_grouped
    preps = []
    for part in calls[0]:
        p = part.to(dev)
        preps.append(ops.gptq_prepare(p.qweight, p.qzeros, p.scales, None, p.bits, p.group_size))
    y = ops.gptq_gemm_grouped(xd, preps)
    ref = og.linear_ref(_np(x), np.concatenate([w["q_proj"], w["k_proj"], w["v_proj"]]), "fp16")
    _check(_np(y.float()), ref, "fp16", f"cfg1 qkv grouped M={m}")
    # o
    y = ops.gptq_gemm(xd, _prep(dev, 1, names.index("o_proj")))
    _check(_np(y.float()), og.linear_ref(_np(x), w["o_proj"], "fp16"), "fp16", f"cfg1 o M={m}")
    # merged gate|up (4096 -> 28672, the streaming kernels at M <= 32)
    gu = calls[2][0].to(dev)
    pgu = ops.gptq_prepare(gu.qweight, gu.qzeros, gu.scales, None, gu.bits, gu.group_size)
    y = ops.gptq_gemm(xd, pgu)
    ref = og.linear_ref(_np(x), np.concatenate([w["gate_proj"], w["up_proj"]]), "fp16")
    _check(_np(y.float()), ref, "fp16", f"cfg1 gate|up M={m}")
    # down (14336 -> 4096, 2-bit), input of the gate|up width's half
    xdn = synth.activations(m, 14336, torch.float16, seed=1300 + m)
    y = ops.gptq_gemm(xdn.to(dev), _prep(dev, 1, names.index("down_proj")))
    _check(_np(y.float()), og.linear_ref(_np(xdn), w["down_proj"], "fp16"), "fp16", f"cfg1 down M={m}")
    assert cases["down_proj"].bits == 2


@pytest.mark.parametrize("m", [1, 16, 64, 256])
@pytest.mark.parametrize("idx", range(3))
def test_config2_act_order(dev, idx, m):
    """Qwen3-8B gate/up/down, 3-bit, act-order (g_idx a seeded permutation)."""
    assert _case(2, idx).g_idx is not None
    x, y = _run(dev, 2, idx, m, "fp16", seed=2000 + 10 * idx + m)
    name = synth.CONFIG2[idx][0]
    _check(_np(y.float()), og.linear_ref(_np(x), _oracle_w(2, idx, "fp16"), "fp16"), "fp16", f"cfg2 {name} M={m}")


# ------------------------------------------------------------------------------ config 4


def _plan(cfg, idx, m):
    c = _case(cfg, idx)
    return N.describe_gptq_plan(m, c.in_features, c.out_features, c.bits, c.group_size, c.g_idx is not None)


@pytest.mark.parametrize("idx", range(4))
def test_config4_m2048(dev, idx):
    """Qwen3-14B prefill shapes at M = 2048, bf16, whole outputs.  The plan is the 256-row tile
    GEMM; gate_up (136 column blocks x 8 row blocks = 1088 tiles) also cuts its last 64 tiles
    along K (fp32 partials + fixup) and takes the XCD-ordered tile map (8 | row blocks)."""
    name = synth.CONFIG4[idx][0]
    plan = _plan(4, idx, 2048)
    print(f"cfg4 {name} M=2048 plan: {plan}")
    assert plan.startswith("k_gemm mt=4"), plan
    if name == "gate_up_proj" and N.load() and torch.cuda.get_device_properties(0).multi_processor_count == 256:
        assert int(re.search(r"split_tiles=(\d+)", plan).group(1)) > 0, plan
    x, y = _run(dev, 4, idx, 2048, "bf16", seed=4000 + idx)
    ref = og.linear_ref(_xin(x, "bf16"), _oracle_w(4, idx, "bf16"), "bf16")
    _check(_np(y.float()), ref, "bf16", f"cfg4 {name} M=2048")


@pytest.mark.parametrize("m", [4096, 8192])
@pytest.mark.parametrize("idx", range(4))
def test_config4_large_m_sampled(dev, idx, m):
    """M = 4096 / 8192: one row of every 256-row block over all columns, and every row over 384
    sampled columns (the last column block included)."""
    name = synth.CONFIG4[idx][0]
    print(f"cfg4 {name} M={m} plan: {_plan(4, idx, m)}")
    x, y = _run(dev, 4, idx, m, "bf16", seed=4100 + 10 * idx + m // 1024)
    w = _oracle_w(4, idx, "bf16")
    xb = _xin(x, "bf16")
    yf = _np(y.float())
    rows = np.array([256 * i + (37 * i) % 256 for i in range(m // 256)])
    _check(yf[rows], og.linear_ref(xb[rows], w, "bf16"), "bf16", f"cfg4 {name} M={m} row sample")
    n = w.shape[0]
    rng = np.random.default_rng(m + idx)
    cols = np.unique(np.concatenate([rng.choice(n - 256, 256, replace=False), np.arange(n - 128, n)]))
    _check(yf[:, cols], og.linear_ref(xb, w[cols], "bf16"), "bf16", f"cfg4 {name} M={m} column sample")


# ------------------------------------------------------------------------------ config 3


def _dbf(dev, idx, seed=0):
    name, k, n = synth.CONFIG3[idx]
    c = synth.dbf_case(name, k, n, 1.0, seed=seed + idx)
    cd = c.to(dev)
    prep = dbf_ops.dbf_prepare(cd.s0, cd.bp1, cd.s2, cd.bp3, cd.s4, k, c.mid, n)
    return c, prep


@pytest.mark.parametrize("m", [1, 32, 512])
@pytest.mark.parametrize("idx", range(2))
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_config3_dbf(dev, idx, m, dtype):
    """DBF at 4096 -> 14336 and 14336 -> 4096 (r = 3185); bf16 as the GemLite path runs it (the
    fp16 scalings cast to bf16, vllm_plugin.py:286-292)."""
    c, prep = _dbf(dev, idx)
    assert c.mid == 3185
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    x = synth.activations(m, c.in_features, td, seed=3000 + 10 * idx + m)
    y = dbf_ops.dbf_forward(x.to(dev), [prep])
    torch.cuda.synchronize()
    sc = [_np(v) for v in (c.s0, c.s2, c.s4)]
    if dtype == "bf16":
        sc = [og.f32_to_bf16_bits(v.astype(np.float32)) for v in sc]
    ref = od.dbf_forward(_xin(x, dtype), sc[0], _np(c.bp1), sc[1], _np(c.bp3), sc[2], c.in_features, c.mid,
                         c.out_features, dtype=dtype)
    _check(_np(y.float()), ref, dtype, f"cfg3 dbf {c.name} {dtype} M={m}")


@pytest.mark.parametrize("m", [1, 32, 512])
@pytest.mark.parametrize("idx", range(2))
def test_config3_mdbf_two_paths(dev, idx, m):
    """MDBF with P = 2 paths of l = 1 at both MLP shapes: path p is a DBF factorisation with
    A_amp = scaling4, Q_U = scaling2, Q_V = 1, B_amp = scaling0 (mdbf_layer.py:278-290)."""
    paths, preps = [], []
    for p in range(2):
        name, k, n = synth.CONFIG3[idx]
        c = synth.dbf_case(name, k, n, 1.0, seed=50 + 2 * idx + p)
        r = c.mid
        path = dict(A_sign_packed=_np(c.bp3), A_shape=(n, r), B_sign_packed=_np(c.bp1), B_shape=(r, k),
                    A_amp=_np(c.s4).reshape(n, 1), B_amp=_np(c.s0).reshape(k, 1),
                    Q_U_amp=_np(c.s2).reshape(r, 1), Q_V_amp=np.ones((r, 1), np.float16))
        paths.append(path)
        t = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(dev)  # noqa: E731
        preps.append(dbf_ops.mdbf_prepare_path(t(path["A_sign_packed"]), path["A_shape"],
                                               t(path["B_sign_packed"]), path["B_shape"], t(path["A_amp"]),
                                               t(path["B_amp"]), t(path["Q_U_amp"]), t(path["Q_V_amp"])))
    x = synth.activations(m, synth.CONFIG3[idx][1], torch.float16, seed=3100 + 10 * idx + m)
    y = dbf_ops.mdbf_forward(x.to(dev), preps)
    torch.cuda.synchronize()
    ref = od.mdbf_forward(_np(x), paths)
    _check(_np(y.float()), ref, "fp16", f"cfg3 mdbf P=2 {synth.CONFIG3[idx][0]} M={m}")
