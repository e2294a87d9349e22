"""FusedMoE dispatch and GPTQMoEMethod's weights and loaders (CPU), restating the expert-config
lookup of vllm_plugins/gptq/vllm_plugin.py:220-283 and the bias loader of
gptoss_wna16_moe.py:27-52 against this package."""

import pytest
import torch

from onecompression_amd import gptq as G
from onecompression_amd import synth
from onecompression_amd.vllm_compat import HAS_VLLM

pytestmark = pytest.mark.skipif(HAS_VLLM, reason="uses the stand-in FusedMoE")

QB = [{
    "self_attn.q_proj": {"bits": 4, "method": "gptq", "group_size": 128},
    "mlp.experts.0.gate_proj": {"bits": 3, "method": "gptq", "group_size": 64},
    "mlp.experts.0.up_proj": {"bits": 3, "method": "gptq", "group_size": 64},
    "mlp.experts.0.down_proj": {"bits": 3, "method": "gptq", "group_size": 64},
}, {
    "self_attn.q_proj": {"bits": 4, "method": "gptq", "group_size": 128},
}, {
    "mlp.experts.3.down_proj": {"bits": 8, "method": "gptq"},
}, {
    "mlp.experts.0.gate_proj": {"bits": 0},
}]


def _cfg():
    return G.MixedGPTQConfig(quantization_bits=QB, group_size=128, desc_act=False, sym=False,
                             checkpoint_format="gptq")


def _moe(layer_idx, E=4, H=128, I=64, **kw):
    from onecompression_amd.vllm_compat import FusedMoE

    return FusedMoE(E, 2, H, I, quant_config=_cfg(), prefix=f"model.layers.{layer_idx}.mlp.experts", **kw)


def test_dispatch_uses_the_expert_entries():
    from onecompression_amd.vllm_compat import FusedMoE

    layer = _moe(0)
    m = layer.quant_method
    assert isinstance(m, G.GPTQMoEMethod)
    assert m.quant_config.weight_bits == 3 and m.quant_config.group_size == 64
    # any expert projection when no gate/up/down of expert 0 is listed; config group size fallback
    m2 = _moe(2).quant_method
    assert m2.quant_config.weight_bits == 8 and m2.quant_config.group_size == 128
    cfg = _cfg()
    stub = FusedMoE.__new__(FusedMoE)
    assert cfg.get_quant_method(stub, "model.layers.1.mlp.experts") is None  # no expert entries
    assert cfg.get_quant_method(stub, "model.layers.3.mlp.experts") is None  # bits 0
    assert cfg.get_quant_method(stub, "model.layers.9.mlp.experts") is None  # beyond the list
    assert cfg.get_quant_method(stub, "lm_head") is None


def test_create_weights_shapes():
    layer = _moe(0, E=4, H=128, I=64, has_bias=True)
    b, g13, g2 = 3, 128 // 64, 64 // 64
    assert layer.w13_qweight.shape == (4, 128 * b // 32, 128)
    assert layer.w13_qzeros.shape == (4, g13, 128 * b // 32)
    assert layer.w13_scales.shape == (4, g13, 128) and layer.w13_scales.dtype == torch.float16
    assert layer.w2_qweight.shape == (4, 64 * b // 32, 128)
    assert layer.w2_qzeros.shape == (4, g2, 128 * b // 32)
    assert layer.w13_bias.shape == (4, 128) and layer.w2_bias.shape == (4, 128)
    assert not hasattr(_moe(0), "w13_bias")
    with pytest.raises(ValueError):
        _moe(0, H=100)


def test_loader_places_gate_up_down_and_bias():
    E, H, I = 3, 128, 64
    layer = _moe(0, E=E, H=H, I=I, has_bias=True)
    cases = {}
    for e in range(E):
        for sid, (k, n) in (("w1", (H, I)), ("w3", (H, I)), ("w2", (I, H))):
            c = synth.gptq_case(sid, k, n, 3, 64, False, seed=10 * e + len(sid) + int(sid[1]))
            cases[e, sid] = c
            pre = "w2" if sid == "w2" else "w13"
            for t in ("qweight", "qzeros", "scales"):
                layer.weight_loader(getattr(layer, f"{pre}_{t}"), getattr(c, t), f"experts.{pre}_{t}", sid, e)
        layer.weight_loader(layer.w13_bias, torch.full((I,), 1.0 + e), "experts.w13_bias", "w1", e)
        layer.weight_loader(layer.w13_bias, torch.full((I,), -1.0 - e), "experts.w13_bias", "w3", e)
        layer.weight_loader(layer.w2_bias, torch.full((H,), 0.5 * e), "experts.w2_bias", "w2", e)
    zw = I * 3 // 32  # 3-bit zero words of one half
    for e in range(E):
        g, u, d = cases[e, "w1"], cases[e, "w3"], cases[e, "w2"]
        assert torch.equal(layer.w13_qweight[e, :, :I], g.qweight) and torch.equal(layer.w13_qweight[e, :, I:], u.qweight)
        assert torch.equal(layer.w13_qzeros[e, :, :zw], g.qzeros) and torch.equal(layer.w13_qzeros[e, :, zw:], u.qzeros)
        assert torch.equal(layer.w13_scales[e, :, I:], u.scales)
        assert torch.equal(layer.w2_qweight[e], d.qweight) and torch.equal(layer.w2_qzeros[e], d.qzeros)
        assert torch.all(layer.w13_bias[e, :I] == 1.0 + e) and torch.all(layer.w13_bias[e, I:] == -1.0 - e)
        assert torch.all(layer.w2_bias[e] == 0.5 * e)
    with pytest.raises(ValueError):  # a down tensor offered as gate
        layer.weight_loader(layer.w13_qweight, cases[0, "w2"].qweight, "experts.w13_qweight", "w1", 0)
    with pytest.raises(ValueError):
        layer.weight_loader(layer.w2_qweight, cases[0, "w2"].qweight, "experts.w2_qweight", "w1", 0)
    assert layer.weight_loader(layer.w2_bias, torch.zeros(H), "experts.w2_bias", "w2", 1, return_success=True)


def test_apply_before_processing():
    layer = _moe(0)
    x = torch.zeros(1, 128, dtype=torch.float16)
    with pytest.raises(RuntimeError):
        layer(x, torch.ones(1, 2), torch.zeros(1, 2, dtype=torch.int32))


def test_act_order_g_idx_params_and_loader():
    """desc_act registers w13_g_idx [E, H] (gate and up share a row, which must agree) and
    w2_g_idx [E, I]."""
    from onecompression_amd.vllm_compat import FusedMoE

    cfg = G.MixedGPTQConfig(quantization_bits=QB, group_size=128, desc_act=True, sym=False, checkpoint_format="gptq")
    E, H, I = 4, 128, 64
    layer = FusedMoE(E, 2, H, I, quant_config=cfg, prefix="model.layers.0.mlp.experts")
    assert tuple(layer.w13_g_idx.shape) == (E, H) and layer.w13_g_idx.dtype == torch.int32
    assert tuple(layer.w2_g_idx.shape) == (E, I)
    g = synth.gptq_case("g", H, I, 3, 64, True, seed=1).g_idx
    layer.weight_loader(layer.w13_g_idx, g, "experts.w13_g_idx", "w1", 2)
    layer.weight_loader(layer.w13_g_idx, g, "experts.w13_g_idx", "w3", 2)  # same order: accepted
    assert torch.equal(layer.w13_g_idx.data[2], g)
    with pytest.raises(ValueError, match="g_idx differ"):
        layer.weight_loader(layer.w13_g_idx, torch.flip(g, [0]), "experts.w13_g_idx", "w3", 2)
    d = synth.gptq_case("d", I, H, 3, 64, True, seed=2).g_idx
    layer.weight_loader(layer.w2_g_idx, d, "experts.w2_g_idx", "w2", 1)
    assert torch.equal(layer.w2_g_idx.data[1], d)


def test_prepare_experts_rejects_differing_gate_up_order():
    from onecompression_amd import moe

    g = synth.gptq_case("g", 128, 64, 4, 64, True, seed=3)
    u = synth.gptq_case("u", 128, 64, 4, 64, True, seed=4)
    d = synth.gptq_case("d", 64, 128, 4, 64, True, seed=5)
    t = lambda c: (c.qweight, c.qzeros, c.scales, c.g_idx)  # noqa: E731
    with pytest.raises(ValueError, match="same g_idx"):
        moe.prepare_experts([t(g)], [t(u)], [t(d)], 4, 64)
