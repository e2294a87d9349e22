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
    assert isinstance(m, G.GPTQLinearMethod) and m.quant_config.weight_bits == 2


def test_dispatch_per_module_group_size():
    cfg = _cfg()
    m = cfg.get_quant_method(_layer(), "model.layers.0.self_attn.o_proj")
    assert isinstance(m, G.GPTQLinearMethod) and m.quant_config.group_size == 128
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
    assert isinstance(m, ROT.RotatedLinearMethod) and isinstance(m.base_method, G.GPTQLinearMethod)
    assert m.fp32_had
    assert isinstance(cfg.get_quant_method(_layer(), "model.layers.0.mlp.up_proj"), G.GPTQLinearMethod)
    plain = G.MixedGPTQConfig.from_config({"quantization_bits": QB})
    assert isinstance(plain.get_quant_method(_layer(), "model.layers.0.mlp.down_proj"), G.GPTQLinearMethod)


def test_rotated_wrapper_installs_one_pre_hook():
    from onecompression_amd import rotation as ROT

    base = G.GPTQLinearMethod(G.GPTQLayerConfig(4, 128, False, False, "gptq"))
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
    method = G.GPTQLinearMethod(G.GPTQLayerConfig(bits, gs, False, False, "gptq"))
    layer = torch.nn.Module()
    method.create_weights(layer, 1024, [256, 64, 64], 1024, 384, torch.float16)
    g = 1024 // 128 if gs == 128 else 1
    assert layer.qweight.shape == (1024 * bits // 32, 384) and layer.qweight.dtype == torch.int32
    assert layer.qzeros.shape == (g, 384 * bits // 32)
    assert layer.scales.shape == (g, 384) and layer.scales.dtype == torch.float16
    assert layer.g_idx.tolist() == [i // (128 if gs == 128 else 1024) for i in range(1024)]


def test_fused_weight_loader_places_shards():
    bits = 4
    method = G.GPTQLinearMethod(G.GPTQLayerConfig(bits, 128, False, False, "gptq"))
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
