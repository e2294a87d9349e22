"""Pins of the MoE oracle (oracle/moe.py) against independent formulations (CPU)."""

import numpy as np
import pytest

from oracle import moe as om


def _experts(rng, E, H, I, bias=False):
    out = []
    for _ in range(E):
        ex = {"gate": rng.normal(0, 0.1, (I, H)).astype(np.float32),
              "up": rng.normal(0, 0.1, (I, H)).astype(np.float32),
              "down": rng.normal(0, 0.1, (H, I)).astype(np.float32)}
        if bias:
            ex.update(gate_bias=rng.normal(0, 0.1, I).astype(np.float32),
                      up_bias=rng.normal(0, 0.1, I).astype(np.float32),
                      down_bias=rng.normal(0, 0.1, H).astype(np.float32))
        out.append(ex)
    return out


def _dense(x, idx, w, experts, act, alpha=1.702, limit=7.0):
    """Token by token, slot by slot, float64, no intermediate rounding."""
    y = np.zeros(x.shape, np.float64)
    for t in range(x.shape[0]):
        for j in range(idx.shape[1]):
            e = int(idx[t, j])
            if e < 0 or e >= len(experts):
                continue
            ex = experts[e]
            g = ex["gate"].astype(np.float64) @ x[t] + ex.get("gate_bias", 0.0)
            u = ex["up"].astype(np.float64) @ x[t] + ex.get("up_bias", 0.0)
            if act == "silu":
                h = g / (1 + np.exp(-g)) * u
            elif act == "gelu_tanh":
                h = 0.5 * g * (1 + np.tanh(np.sqrt(2 / np.pi) * (g + 0.044715 * g ** 3))) * u
            else:
                gc = np.minimum(g, limit)
                uc = np.clip(u, -limit, limit)
                h = (uc + 1) * gc / (1 + np.exp(-alpha * gc))
            y[t] += w[t, j] * (ex["down"].astype(np.float64) @ h + ex.get("down_bias", 0.0))
    return y


@pytest.mark.parametrize("act,bias", [("silu", False), ("gelu_tanh", False), ("gpt_oss", True)])
def test_moe_oracle_matches_dense_formulation(act, bias):
    rng = np.random.default_rng(3)
    E, H, I, M, k = 5, 64, 32, 6, 2
    ex = _experts(rng, E, H, I, bias)
    x = rng.normal(0, 1, (M, H)).astype(np.float16).astype(np.float32)
    idx = rng.integers(0, E, (M, k))
    idx[0] = [2, 2]        # the same expert twice in one token counts twice
    idx[1, 1] = -1         # an invalid slot contributes nothing
    w = rng.random((M, k)).astype(np.float32)
    got = om.moe_forward(x, idx, w, ex, act)
    ref = _dense(x, idx, w, ex, act)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) < 5e-3
    # a planted routing mistake (weights of the other slot) is caught
    bad = om.moe_forward(x, idx, w[:, ::-1].copy(), ex, act)
    assert np.max(np.abs(bad - ref)) / np.max(np.abs(ref)) > 5e-2


def test_gpt_oss_combine_special_points():
    a, lim = 1.702, 7.0
    # gate = 0 -> glu = 0; gate clamped to the limit; up clamped to +-limit
    assert om.gpt_oss_combine([0.0], [3.0], a, lim, "fp16")[0] == 0.0
    big = om.gpt_oss_combine([100.0], [100.0], a, lim, "fp16")[0]
    sig = np.float16(1.0 / (1.0 + np.exp(-np.float16(lim * a))))
    want = np.float16(np.float16(lim + 1.0) * np.float16(np.float16(lim) * sig))
    assert big == np.float32(want)
    neg = om.gpt_oss_combine([1.0], [-100.0], a, lim, "fp16")[0]
    assert neg < 0 and abs(neg - (-lim + 1) * 1.0 / (1 + np.exp(-a))) < 2e-2
    # sigmoid(0) = 1/2 in silu: silu(x) ~ x/2 near 0
    assert abs(om.silu([1e-3], "fp16")[0] - 5e-4) < 1e-6
