"""GPU: the online Hadamard kernel and the rotated down_proj plugin path against the oracle."""

import numpy as np
import pytest
import torch

from oracle import gptq as og
from oracle import hadamard as oh
from onecompression_amd import gptq as G
from onecompression_amd import ops, synth
from onecompression_amd.vllm_compat import HAS_VLLM, LinearBase

pytestmark = pytest.mark.gpu


def _x(m, n, dtype, seed):
    return torch.randn(m, n, generator=torch.Generator().manual_seed(seed)).to(dtype)


def _f32(t, dtype):
    return t.float().numpy() if dtype == torch.float16 else t.float().numpy()


@pytest.mark.parametrize("n", [14336, 12288, 17408, 4096, 24, 320, 2 * 140, 20, 4, 1, 32768, 27648, 28672,
                               2240, 2304, 3840, 2432,  # blocks of 140, 36, 60, 76 (L >= 16)
                               11008, 9984, 25600, 6656, 832, 2752, 2496])  # Williamson 172, 156, 100, 52 (+ L = 16)
@pytest.mark.parametrize("m", [1, 3, 64])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rounding", ["once", "fp32"])
def test_hadamard_matches_oracle(dev, n, m, dtype, rounding):
    x = _x(m, n, dtype, n + m)
    y = ops.hadamard(x.to(dev), rounding=rounding).cpu()
    xf = x.float().numpy()
    ref = oh.online_hadamard(xf)
    # Against the float64 transform: "once" rounds the transform and u = RNE(.) / sqrt(n) (K > 1:
    # their errors reach y_i through sum_c |H[i, c]| |u_c| = sum_c |u_c|) and the fp32-accumulated
    # result; "fp32" rounds the result only (u carried to 22-24 bits).
    ulp = 2.0 ** (-10 if dtype == torch.float16 else -7)
    K = oh.pick_order(n)
    mid = 0.0
    if K > 1:
        u = np.abs(oh.fwht(xf.reshape(m, K, n // K)) / np.sqrt(n))
        mid = np.broadcast_to(u.sum(axis=1, keepdims=True), u.shape).reshape(m, n)
    err = np.abs(y.float().numpy() - ref)
    bound = ulp * np.maximum(np.abs(ref), 2.0 ** -14) + (ulp if rounding == "once" else 2.0 ** -20) * mid + 1e-6
    assert np.all(err <= bound), float((err / bound).max())


def _spacing(v, dtype):
    """One unit in the last place of the output dtype at v."""
    if dtype == torch.float16:
        return np.spacing(np.abs(v).astype(np.float16)).astype(np.float64)
    b = og.f32_to_bf16_bits(np.abs(v).astype(np.float32)).astype(np.uint32)
    lo = og.bf16_bits_to_f32(b).astype(np.float64)
    hi = og.bf16_bits_to_f32(b + 1).astype(np.float64)
    return hi - lo


# Every rounding sequence of the reference (rotation.py:100-112) through both kernels (M <= 16
# products, M > 16 one workgroup per row; "stages" always the latter) against the oracle's
# restatement, which takes the transform's and the H_K product's sums exact: outputs equal bit for
# bit except where the kernel's fp32 sums round.  Such a rounding moves y by at most one ulp of y
# (two where "once" rounds a transform sum that sat at a tie) plus, through the H_K mix, what it
# moved u: one ulp of u for "once", 2^-10 ulp of u where u is carried in fp32 or exact.
@pytest.mark.parametrize("n", [14336, 12288, 4096, 11008, 20, 4])
@pytest.mark.parametrize("m", [1, 3, 40])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rounding", ["stages", "once", "fp32"])
def test_hadamard_rounding_sequences(dev, n, m, dtype, rounding):
    x = _x(m, n, dtype, 3 * n + m)
    y = ops.hadamard(x.to(dev), rounding=rounding).cpu().float().numpy().astype(np.float64)
    dt = "fp16" if dtype == torch.float16 else "bf16"
    ref = oh.online_hadamard_rounded(x.float().numpy(), dt, rounding)
    K = oh.pick_order(n)
    u_sp = 0.0
    if K > 1:  # largest ulp of u = FWHT_L / sqrt(n) in each row
        u = np.abs(oh.fwht(x.float().numpy().reshape(m, K, n // K)) / np.sqrt(n)).max(axis=(1, 2))
        u_sp = _spacing(u, dtype)[:, None] * (1.0 if rounding == "once" else 2.0 ** -10)
    diff = np.abs(y - ref)
    # "once": a transform rounded the other way at a tie moves y by about one ulp of y before y's
    # own rounding (K = 1), or by one ulp of u through the mix.  Outputs far below the row's
    # magnitude (cancellation) also carry the fp32 sums' absolute error, 2^-18 of the row's largest.
    fp32_abs = 2.0 ** -18 * np.abs(ref).max(axis=1, keepdims=True)
    bound = (2.0 if rounding == "once" else 1.0) * _spacing(ref, dtype) + u_sp + fp32_abs
    assert np.all(diff <= bound), float((diff / bound).max())
    # "fp32" carries u in two (fp16) parts, 22 bits: near-ties of y flip more often at K = 172
    assert np.mean(diff > 0) <= (1e-2 if rounding == "fp32" else 2e-3), float(np.mean(diff > 0))


# Known answers derived by hand (fp16 [2048, 1, 1, 1], bf16 [256, 1, 1, 1]: the first stage's
# 2048 + 1 rounds to 2048; the exact sum 2051 rounds to 2052; 2051 / 2 = 1025.5 rounds to 1026).
@pytest.mark.parametrize("dtype,x,want", [
    (torch.float16, [2048, 1, 1, 1], {"stages": [1025, 1023.5, 1023, 1023.5], "once": [1026, 1023.5, 1023.5, 1023.5],
                                      "fp32": [1026, 1023.5, 1023.5, 1023.5]}),
    (torch.bfloat16, [256, 1, 1, 1], {"stages": [129, 127.5, 127, 127.5], "once": [130, 127.5, 127.5, 127.5],
                                      "fp32": [130, 127.5, 127.5, 127.5]})])
def test_hadamard_rounding_known_answers(dev, dtype, x, want):
    xt = torch.tensor([x], dtype=dtype, device=dev)
    for rounding, w in want.items():
        assert ops.hadamard(xt, rounding=rounding).float().cpu().tolist() == [w], rounding


def test_hadamard_in_place_and_strided(dev):
    n = 14336
    base = _x(4, n + 64, torch.float16, 1).to(dev)
    x = base[:, :n]                    # row stride n + 64
    want = ops.hadamard(x.contiguous())
    out = torch.empty((4, n), dtype=torch.float16, device=dev)
    got = ops.hadamard(x, out=out)
    assert torch.equal(got, want)
    y = x.contiguous()
    ops.hadamard(y, out=y)            # aliasing output and input
    assert torch.equal(y, want)


def test_hadamard_rejects_bad_n(dev):
    with pytest.raises(ValueError):
        ops.hadamard(torch.zeros(1, 1000, dtype=torch.float16, device=dev))


@pytest.mark.skipif(HAS_VLLM, reason="layer built with the local LinearBase stand-in")
@pytest.mark.parametrize("m,fp32_had", [(1, False), (7, False), (130, False), (1, True), (130, True)])
def test_rotated_down_proj_layer(dev, m, fp32_had):
    """rotated: true -> the down_proj input is Hadamard-transformed before the GPTQ GEMM, rounded as
    the config's fp32_had asks."""
    k, n = 14336, 512
    qb = [{"mlp.down_proj": {"bits": 4, "method": "gptq", "group_size": 128}}]
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": qb, "checkpoint_format": "gptq",
                                         "rotated": True, "fp32_had": fp32_had})
    layer = LinearBase(k, n, quant_config=cfg, prefix="model.layers.0.mlp.down_proj")
    c = synth.gptq_case("down", k, n, 4, 128, False, seed=5)
    for name in ("qweight", "qzeros", "scales"):
        p = getattr(layer, name)
        p.weight_loader(p, getattr(c, name))
    layer.to(dev)
    layer.quant_method.process_weights_after_loading(layer)
    x = synth.activations(m, k, seed=6)
    y = layer(x.to(dev)).float().cpu().numpy()
    xh = oh.online_hadamard_rounded(x.float().numpy(), "fp16", "fp32" if fp32_had else "stages").astype(np.float16)
    w = og.dequantize(c.qweight.numpy(), c.qzeros.numpy(), c.scales.numpy(), og.default_g_idx(k, 128), 4,
                      "gptq", "fp16")
    ref = og.linear_ref(xh, w, "fp16")
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) <= 1e-2
