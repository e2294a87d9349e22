"""Mixed-GPTQ plugin surface (CPU): config parsing, per-module dispatch and
create_weights, restating tests/vllm_plugins/gptq/test_mixed_gptq.py:184-348
and tests/vllm_plugins/test_module_attn_alias.py against this package."""

import pytest
import torch

from onecompression_amd import gptq as G
from onecompression_amd import module_utils as MU
from onecompression_amd.vllm_compat import HAS_VLLM, LinearBase, UnquantizedLinearMethod

QB = [{
    "self_attn.q_proj": {"bits": 4, "method": "gptq", "group_size": 128},
    "self_attn.k_proj": {"bits": 4, "method": "gptq", "group_size": 128},
    "self_attn.v_proj": {"bits": 4, "method": "gptq", "group_size": 128},
    "self_attn.o_proj": {"bits": 4, "method": "gptq", "group_size": 128},
    "mlp.gate_proj": {"bits": 2, "method": "gptq", "group_size": 32},
    "mlp.up_proj": {"bits": 2, "method": "gptq", "group_size": 32},
    "mlp.down_proj": {"bits": 2, "method": "gptq", "group_size": 32},
}]


def _cfg(qb=None, gs=-1, **kw):
    return G.MixedGPTQConfig(quantization_bits=qb or QB, group_size=gs, desc_act=False, sym=True, **kw)


class _Lin(LinearBase if not HAS_VLLM else torch.nn.Module):
    def __init__(self):  # a LinearBase instance without building weights
        torch.nn.Module.__init__(self)


def _layer():
    return _Lin.__new__(_Lin) if HAS_VLLM else _Lin()


def test_group_size_priority():
    cfg = _cfg(gs=256)
    assert cfg.resolve_group_size({"bits": 4, "group_size": 128}) == 128
    assert cfg.resolve_group_size({"bits": 4, "params": {"group_size": 64}}) == 64
    assert cfg.resolve_group_size({"bits": 4, "group_size": 128, "params": {"group_size": 64}}) == 128
    assert cfg.resolve_group_size({"bits": 4}) == 256
    assert cfg.resolve_group_size(None) == 256


def test_from_config_round_trip_and_defaults():
    cfg = G.MixedGPTQConfig.from_config({"quant_method": "mixed_gptq", "quantization_bits": QB,
                                         "group_size": -1, "desc_act": False, "sym": True})
    assert cfg.group_size == -1 and cfg.sym is True and len(cfg.quantization_bits) == 1
    assert cfg.checkpoint_format == "gptq_v2"  # vllm_plugin.py:154 default when the key is absent
    assert G.MixedGPTQConfig.from_config({"quantization_bits": QB, "checkpoint_format": "gptq"}
                                         ).checkpoint_format == "gptq"
    assert G.MixedGPTQConfig.get_name() == "mixed_gptq"
    assert G.MixedGPTQConfig.get_supported_act_dtypes() == [torch.half, torch.bfloat16]


def test_legacy_layer_bits():
    cfg = G.MixedGPTQConfig.from_config({"layer_bits": [4, 4, 2], "group_size": 128})
    assert len(cfg.quantization_bits) == 3 and cfg.group_size == 128
    m = cfg.get_quant_method(_layer(), "model.layers.2.mlp.down_proj")
    assert isinstance(m, G.MixedGPTQLinearMethod) and m.quant_config.weight_bits == 2


def test_dispatch_per_module_group_size():
    cfg = _cfg()
    m = cfg.get_quant_method(_layer(), "model.layers.0.self_attn.o_proj")
    assert isinstance(m, G.MixedGPTQLinearMethod) and m.quant_config.group_size == 128
    m = cfg.get_quant_method(_layer(), "model.layers.0.mlp.down_proj")
    assert m.quant_config.group_size == 32 and m.quant_config.weight_bits == 2


def test_non_linear_and_non_layer_prefixes():
    cfg = _cfg()
    assert cfg.get_quant_method(torch.nn.ReLU(), "model.layers.0.self_attn.o_proj") is None
    assert isinstance(cfg.get_quant_method(_layer(), "model.embed_tokens"), UnquantizedLinearMethod)
    assert isinstance(cfg.get_quant_method(_layer(), "model.layers.5.mlp.down_proj"), UnquantizedLinearMethod)
    assert isinstance(cfg.get_quant_method(_layer(), "vision_tower.layers.0.mlp.down_proj"),
                      UnquantizedLinearMethod)


def test_bits_zero_and_unknown_method_are_unquantized():
    qb = [{"mlp.down_proj": {"bits": 0}, "mlp.up_proj": {"bits": 4, "method": "rtn_fancy"}}]
    cfg = _cfg(qb)
    assert isinstance(cfg.get_quant_method(_layer(), "model.layers.0.mlp.down_proj"), UnquantizedLinearMethod)
    assert isinstance(cfg.get_quant_method(_layer(), "model.layers.0.mlp.up_proj"), UnquantizedLinearMethod)


def test_fused_module_resolution_and_mismatch():
    cfg = _cfg()
    m = cfg.get_quant_method(_layer(), "model.layers.0.self_attn.qkv_proj")
    assert m.quant_config.weight_bits == 4
    mixed = [{"self_attn.q_proj": {"bits": 4}, "self_attn.k_proj": {"bits": 8}, "self_attn.v_proj": {"bits": 8}}]
    with pytest.raises(ValueError, match="All shards of fused layers"):
        _cfg(mixed).get_quant_method(_layer(), "model.layers.0.self_attn.qkv_proj")
    partial = [{"mlp.gate_proj": {"bits": 4}}]
    with pytest.raises(ValueError):
        _cfg(partial).get_quant_method(_layer(), "model.layers.0.mlp.gate_up_proj")


def test_attn_alias():
    assert MU.normalize_module_suffix("attn.o_proj") == "self_attn.o_proj"
    assert MU.normalize_module_suffix("mlp.gate_up_proj") == "mlp.gate_up_proj"
    qb = [{"self_attn.o_proj": {"bits": 4, "method": "gptq", "params": {"group_size": -1}}}]
    assert MU.lookup_module_config(qb, 0, "attn.o_proj")["bits"] == 4


def test_rotated_down_proj_is_wrapped():
    """rotation.py:242-261: only mlp.down_proj of a rotated checkpoint gets the online Hadamard."""
    from onecompression_amd import rotation as ROT

    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": QB, "rotated": True, "fp32_had": True})
    m = cfg.get_quant_method(_layer(), "model.layers.0.mlp.down_proj")
    assert isinstance(m, ROT.RotatedLinearMethod) and isinstance(m.base_method, G.MixedGPTQLinearMethod)
    assert m.fp32_had
    assert isinstance(cfg.get_quant_method(_layer(), "model.layers.0.mlp.up_proj"), G.MixedGPTQLinearMethod)
    plain = G.MixedGPTQConfig.from_config({"quantization_bits": QB})
    assert isinstance(plain.get_quant_method(_layer(), "model.layers.0.mlp.down_proj"), G.MixedGPTQLinearMethod)


def test_rotated_wrapper_installs_one_pre_hook():
    from onecompression_amd import rotation as ROT

    base = G.MixedGPTQLinearMethod(G.GPTQLayerConfig(4, 128, False, False, "gptq"))
    m = ROT.RotatedLinearMethod(base, fp32_had=False)
    layer = torch.nn.Module()
    m.create_weights(layer, 256, [64], 256, 64, torch.float16)
    m.create_weights(layer, 256, [64], 256, 64, torch.float16)
    assert layer._onecomp_hadamard_prehook_installed and len(layer._forward_pre_hooks) == 1
    tp = torch.nn.Module()
    tp.tp_size, tp.input_is_parallel = 2, True
    with pytest.raises(NotImplementedError, match="all-gather"):
        m.create_weights(tp, 256, [64], 256, 64, torch.float16)


@pytest.mark.parametrize("bits", [2, 3, 4, 8])
@pytest.mark.parametrize("gs", [128, -1])
def test_create_weights_shapes(bits, gs):
    method = G.MixedGPTQLinearMethod(G.GPTQLayerConfig(bits, gs, False, False, "gptq"))
    layer = torch.nn.Module()
    method.create_weights(layer, 1024, [256, 64, 64], 1024, 384, torch.float16)
    g = 1024 // 128 if gs == 128 else 1
    assert layer.qweight.shape == (1024 * bits // 32, 384) and layer.qweight.dtype == torch.int32
    assert layer.qzeros.shape == (g, 384 * bits // 32)
    assert layer.scales.shape == (g, 384) and layer.scales.dtype == torch.float16
    assert layer.g_idx.tolist() == [i // (128 if gs == 128 else 1024) for i in range(1024)]


def test_fused_weight_loader_places_shards():
    bits = 4
    method = G.MixedGPTQLinearMethod(G.GPTQLayerConfig(bits, 128, False, False, "gptq"))
    layer = torch.nn.Module()
    method.create_weights(layer, 256, [64, 32, 32], 256, 128, torch.float16)
    parts = {"q": 64, "k": 32, "v": 32}
    off = 0
    for sid, n in parts.items():
        qw = torch.full((256 * bits // 32, n), hash(sid) % 1000, dtype=torch.int32)
        layer.qweight.weight_loader(layer.qweight, qw, sid)
        qz = torch.full((2, n * bits // 32), hash(sid) % 777, dtype=torch.int32)
        layer.qzeros.weight_loader(layer.qzeros, qz, sid)
        assert torch.equal(layer.qweight.data[:, off:off + n], qw)
        assert torch.equal(layer.qzeros.data[:, off * bits // 32:(off + n) * bits // 32], qz)
        off += n


MIXED_QKV = [{"self_attn.q_proj": {"bits": 4, "method": "gptq", "group_size": 128},
              "self_attn.k_proj": {"bits": 8, "method": "gptq", "group_size": 128},
              "self_attn.v_proj": {"bits": 8, "method": "gptq", "group_size": 64}}]


def test_fused_mixed_bits_is_opt_in():
    """Default: the reference's ValueError; with fused_mixed_bits: one method over all shards."""
    with pytest.raises(ValueError, match="All shards of fused layers"):
        G.MixedGPTQConfig.from_config({"quantization_bits": MIXED_QKV}).get_quant_method(
            _layer(), "model.layers.0.self_attn.qkv_proj")
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": MIXED_QKV, "fused_mixed_bits": True})
    m = cfg.get_quant_method(_layer(), "model.layers.0.self_attn.qkv_proj")
    assert isinstance(m, G.MixedFusedGPTQLinearMethod)
    assert [(c.weight_bits, c.group_size) for c in m.part_configs] == [(4, 128), (8, 128), (8, 64)]
    # a missing shard still raises
    partial = [{"mlp.gate_proj": {"bits": 4}}]
    with pytest.raises(ValueError):
        G.MixedGPTQConfig.from_config({"quantization_bits": partial, "fused_mixed_bits": True}).get_quant_method(
            _layer(), "model.layers.0.mlp.gate_up_proj")


def test_fused_mixed_bits_loaders_place_shards():
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": MIXED_QKV, "fused_mixed_bits": True})
    m = cfg.get_quant_method(_layer(), "model.layers.0.self_attn.qkv_proj")
    layer = torch.nn.Module()
    k, parts = 256, [64, 32, 32]
    m.create_weights(layer, k, parts, k, sum(parts), torch.float16)
    loaded = {}
    for i, (sid, n, b, gs) in enumerate(zip("qkv", parts, (4, 8, 8), (128, 128, 64))):
        g = k // gs
        qw = torch.randint(-2**31, 2**31 - 1, (k * b // 32, n), dtype=torch.int32)
        qz = torch.randint(-2**31, 2**31 - 1, (g, n * b // 32), dtype=torch.int32)
        sc = torch.rand(g, n).half()
        gi = torch.randperm(k).to(torch.int32) // gs
        for name, t in (("qweight", qw), ("qzeros", qz), ("scales", sc), ("g_idx", gi)):
            p = getattr(layer, name)
            p.weight_loader(p, t, sid)
        loaded[i] = (qw, qz, sc, gi)
        with pytest.raises(ValueError):
            layer.qweight.weight_loader(layer.qweight, qw[:, :1], sid)
    for i in range(3):
        for got, want in zip(m.shard_tensors(layer, i), loaded[i]):
            assert torch.equal(got, want)


# ---------------------------------------------------------------- weight-loader selection
# vLLM hands a linear layer's params the v2 weight loader when the quant method's class name is on
# WEIGHT_LOADER_V2_SUPPORTED, else the v1 loader (vllm_plugins/utils/rotation.py:126-144).  The
# stand-in LinearBase makes the same choice; these tests hold the plugin to it.

@pytest.mark.skipif(HAS_VLLM, reason="exercises the stand-in LinearBase's loader selection")
def test_gptq_method_gets_the_v1_loader_and_loads_fused_shards():
    from onecompression_amd import synth
    from onecompression_amd.vllm_compat import WEIGHT_LOADER_V2_SUPPORTED

    assert "GPTQLinearMethod" in WEIGHT_LOADER_V2_SUPPORTED  # vLLM's own GPTQ method takes v2
    assert "MixedGPTQLinearMethod" not in WEIGHT_LOADER_V2_SUPPORTED
    qb = [{"self_attn.q_proj": {"bits": 3, "method": "gptq", "group_size": 128},
           "self_attn.k_proj": {"bits": 3, "method": "gptq", "group_size": 128},
           "self_attn.v_proj": {"bits": 3, "method": "gptq", "group_size": 128}}]
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": qb, "checkpoint_format": "gptq"})
    sizes = [128, 64, 64]
    layer = LinearBase(256, 256, quant_config=cfg, prefix="model.layers.0.self_attn.qkv_proj",
                       output_partition_sizes=sizes)
    assert layer.loader_version == 1
    shards = [synth.gptq_case(s, 256, n, 3, 128, False, seed=i) for i, (s, n) in enumerate(zip("qkv", sizes))]
    for sid, c in zip("qkv", shards):
        for name in ("qweight", "qzeros", "scales"):
            p = getattr(layer, name)
            p.weight_loader(p, getattr(c, name), sid)
    assert torch.equal(layer.qweight.data, torch.cat([c.qweight for c in shards], 1))
    assert torch.equal(layer.qzeros.data, torch.cat([c.qzeros for c in shards], 1))  # packed along N
    assert torch.equal(layer.scales.data, torch.cat([c.scales for c in shards], 1))


@pytest.mark.skipif(HAS_VLLM, reason="exercises the stand-in LinearBase's loader selection")
def test_a_v2_listed_name_would_break_plain_parameters():
    """What the method's name avoids: the same create_weights under vLLM's GPTQ method name gets
    the v2 loader, which plain Parameters cannot serve."""
    named_like_vllm = type("GPTQLinearMethod", (G.MixedGPTQLinearMethod,), {})
    cfg = G.GPTQLayerConfig(4, 128, False, False, "gptq")

    class _Cfg:
        def get_quant_method(self, layer, prefix):
            return named_like_vllm(cfg)

    layer = LinearBase(256, 64, quant_config=_Cfg(), prefix="model.layers.0.mlp.up_proj")
    assert layer.loader_version == 2
    with pytest.raises(AttributeError):
        layer.qweight.weight_loader(layer.qweight, torch.zeros_like(layer.qweight))


@pytest.mark.skipif(HAS_VLLM, reason="exercises the stand-in LinearBase's loader selection")
def test_rotation_wrapper_keeps_the_base_loader_choice():
    """rotation.py:232-261: a v1 base keeps v1 behind RotatedLinearMethod; a v2-native base
    (unquantized down_proj of a rotated checkpoint) gets the listed RotatedLinearMethodV2 and loads
    through its params' own v2 methods."""
    from onecompression_amd import rotation as ROT

    qb = [{"mlp.down_proj": {"bits": 4, "method": "gptq", "group_size": 128},
           "mlp.up_proj": {"bits": 4, "method": "gptq", "group_size": 128}}]
    cfg = G.MixedGPTQConfig.from_config({"quantization_bits": qb, "rotated": True})
    q = LinearBase(256, 64, quant_config=cfg, prefix="model.layers.0.mlp.down_proj")
    assert type(q.quant_method) is ROT.RotatedLinearMethod and q.loader_version == 1
    qb0 = [{"mlp.down_proj": {"bits": 0}}]
    cfg0 = G.MixedGPTQConfig.from_config({"quantization_bits": qb0, "rotated": True})
    u = LinearBase(256, 64, quant_config=cfg0, prefix="model.layers.0.mlp.down_proj")
    assert type(u.quant_method) is ROT.RotatedLinearMethodV2 and u.loader_version == 2
    w = torch.randn(64, 256).half()
    u.weight.weight_loader(u.weight, w)
    assert torch.equal(u.weight.data, w)


def test_moe_expert_entry_preference():
    """vllm_plugin.py:220-239: the first gate_proj entry of the layer's experts, else up, else down,
    else any expert entry; layers past the config have none."""
    qb = [{"mlp.experts.1.down_proj": {"bits": 2}, "mlp.experts.0.up_proj": {"bits": 3},
           "mlp.experts.3.gate_proj": {"bits": 4}, "mlp.experts.2.gate_proj": {"bits": 8}},
          {"mlp.experts.0.down_proj": {"bits": 2}, "mlp.experts.0.w_extra": {"bits": 3}},
          {"mlp.experts.0.w_extra": {"bits": 3}, "self_attn.q_proj": {"bits": 4}}]
    cfg = G.MixedGPTQConfig(quantization_bits=qb)
    assert cfg._lookup_moe_expert_config(0)["bits"] == 4
    assert cfg._lookup_moe_expert_config(1)["bits"] == 2
    assert cfg._lookup_moe_expert_config(2)["bits"] == 3
    assert cfg._lookup_moe_expert_config(3) is None
    assert cfg._resolve_group_size(None) == cfg.group_size
