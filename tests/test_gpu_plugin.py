"""GPU: the Mixed-GPTQ plugin end to end (create_weights -> weight loaders ->
process_weights_after_loading -> apply) against the oracle."""

import numpy as np
import pytest
import torch

from oracle import gptq as og
from onecompression_amd import gptq as G
from onecompression_amd import synth
from onecompression_amd.vllm_compat import HAS_VLLM, LinearBase

pytestmark = [pytest.mark.gpu,
              pytest.mark.skipif(HAS_VLLM, reason="layer built with the local LinearBase stand-in")]


def _ref(cases, x, dtype="fp16"):
    ws = []
    for c in cases:
        g = c.g_idx.numpy() if c.g_idx is not None else og.default_g_idx(c.in_features, c.group_size)
        ws.append(og.dequantize(c.qweight.numpy(), c.qzeros.numpy(), c.scales.numpy(), g, c.bits,
                                "gptq", dtype))
    return og.linear_ref(x, np.concatenate(ws, axis=0), dtype)


def test_fused_qkv_layer(dev):
    qb = [{f"self_attn.{p}_proj": {"bits": 4, "method": "gptq", "group_size": 128} for p in "qkv"}]
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": qb, "checkpoint_format": "gptq"})
    parts = [256, 64, 64]
    layer = LinearBase(1024, sum(parts), quant_config=cfg, prefix="model.layers.0.self_attn.qkv_proj",
                       output_partition_sizes=parts)
    cases = [synth.gptq_case(s, 1024, n, 4, 128, False, seed=i) for i, (s, n) in enumerate(zip("qkv", parts))]
    for c, sid in zip(cases, "qkv"):
        for name in ("qweight", "qzeros", "scales"):
            p = getattr(layer, name)
            p.weight_loader(p, getattr(c, name), sid)
    layer.to(dev)
    layer.quant_method.process_weights_after_loading(layer)
    x = synth.activations(5, 1024, seed=9)
    y = layer(x.to(dev)).float().cpu().numpy()
    ref = _ref(cases, x.numpy())
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) <= 1e-2


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
def test_act_order_down_proj_layer(dev, bits):
    qb = [{"mlp.down_proj": {"bits": bits, "method": "gptq", "params": {"group_size": 128}}}]
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": qb, "desc_act": True,
                                         "checkpoint_format": "gptq"})
    k, n = 2048, 256
    layer = LinearBase(k, n, quant_config=cfg, prefix="model.layers.0.mlp.down_proj")
    c = synth.gptq_case("down", k, n, bits, 128, True, seed=bits)
    for name in ("qweight", "qzeros", "scales", "g_idx"):
        p = getattr(layer, name)
        p.weight_loader(p, getattr(c, name))
    layer.to(dev)
    layer.quant_method.process_weights_after_loading(layer)
    x = synth.activations(3, k, seed=4)
    y = layer(x.to(dev)).float().cpu().numpy()
    ref = _ref([c], x.numpy())
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) <= 1e-2


@pytest.mark.parametrize("v_gs,act,m", [(128, False, 1), (128, True, 4), (64, False, 3), (128, False, 40)])
def test_fused_qkv_mixed_bits_layer(dev, v_gs, act, m):
    """fused_mixed_bits: q@4b, k/v@8b served as one qkv_proj (one launch when every group is a
    multiple of 128 and M <= 16, shard by shard otherwise), with bias, vs the oracle."""
    qb = [{"self_attn.q_proj": {"bits": 4, "method": "gptq", "group_size": 128},
           "self_attn.k_proj": {"bits": 8, "method": "gptq", "group_size": 128},
           "self_attn.v_proj": {"bits": 8, "method": "gptq", "group_size": v_gs}}]
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": qb, "checkpoint_format": "gptq",
                                         "desc_act": act, "fused_mixed_bits": True})
    parts, k = [512, 128, 128], 1024
    layer = LinearBase(k, sum(parts), bias=True, quant_config=cfg, prefix="model.layers.0.self_attn.qkv_proj",
                       output_partition_sizes=parts)
    assert isinstance(layer.quant_method, G.MixedFusedGPTQLinearMethod)
    cases = [synth.gptq_case(s, k, n, b, gs, act, seed=i)
             for i, (s, n, b, gs) in enumerate(zip("qkv", parts, (4, 8, 8), (128, 128, v_gs)))]
    for c, sid in zip(cases, "qkv"):
        for name in ("qweight", "qzeros", "scales") + (("g_idx",) if act else ()):
            p = getattr(layer, name)
            p.weight_loader(p, getattr(c, name), sid)
    bias = (torch.randn(sum(parts), generator=torch.Generator().manual_seed(2)) * 0.1).half()
    layer.bias.data.copy_(bias)
    layer.to(dev)
    layer.quant_method.process_weights_after_loading(layer)
    x = synth.activations(m, k, seed=9)
    y = layer(x.to(dev)).float().cpu().numpy()
    ref = _ref(cases, x.numpy()) + bias.float().numpy()
    assert np.max(np.abs(y - ref)) / np.max(np.abs(ref)) <= 1e-2
