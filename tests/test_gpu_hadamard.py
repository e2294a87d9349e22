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
def test_hadamard_matches_oracle(dev, n, m, dtype):
    x = _x(m, n, dtype, n + m)
    y = ops.hadamard(x.to(dev)).cpu()
    xf = x.float().numpy()
    ref = oh.online_hadamard(xf)
    # Two roundings to the output dtype: of u = FWHT_L / sqrt(n) (K > 1 only),
    # whose error reaches y_i through sum_c |H[i, c]| |u_c| = sum_c |u_c|, and
    # of the fp32-accumulated result.
    ulp = 2.0 ** (-10 if dtype == torch.float16 else -7)
    K = oh.pick_order(n)
    mid = 0.0
    if K > 1:
        u = np.abs(oh.fwht(xf.reshape(m, K, n // K)) / np.sqrt(n))
        mid = np.broadcast_to(u.sum(axis=1, keepdims=True), u.shape).reshape(m, n)
    err = np.abs(y.float().numpy() - ref)
    bound = ulp * np.maximum(np.abs(ref), 2.0 ** -14) + 0.5 * ulp * mid + 1e-6
    assert np.all(err <= bound), float((err / bound).max())


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
@pytest.mark.parametrize("m", [1, 7, 130])
def test_rotated_down_proj_layer(dev, m):
    """rotated: true -> the down_proj input is Hadamard-transformed before the GPTQ GEMM."""
    k, n = 14336, 512
    qb = [{"mlp.down_proj": {"bits": 4, "method": "gptq", "group_size": 128}}]
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": qb, "checkpoint_format": "gptq",
                                         "rotated": True})
    layer = LinearBase(k, n, quant_config=cfg, prefix="model.layers.0.mlp.down_proj")
    c = synth.gptq_case("down", k, n, 4, 128, False, seed=5)
    for name in ("qweight", "qzeros", "scales"):
        p = getattr(layer, name)
        p.weight_loader(p, getattr(c, name))
    layer.to(dev)
    layer.quant_method.process_weights_after_loading(layer)
    x = synth.activations(m, k, seed=6)
    y = layer(x.to(dev)).float().cpu().numpy()
    xh = torch.from_numpy(oh.online_hadamard(x.float().numpy()).astype(np.float32)).half().numpy()
    w = og.dequantize(c.qweight.numpy(), c.qzeros.numpy(), c.scales.numpy(), og.default_g_idx(k, 128), 4,
                      "gptq", "fp16")
    ref = og.linear_ref(xh, w, "fp16")
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) <= 1e-2
