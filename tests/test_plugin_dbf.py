"""DBF plugin surface (CPU): config parsing/dispatch and create_weights,
restating tests/vllm_plugins/dbf/test_dbf_config.py:27-66 and the parameter
layout of vllm_plugins/dbf/vllm_plugin.py:90-230."""

import pytest
import torch

from oracle import dbf as od
from onecompression_amd import dbf as D
from onecompression_amd.vllm_compat import HAS_VLLM, LinearBase, UnquantizedLinearMethod


class _Lin(LinearBase if not HAS_VLLM else torch.nn.Module):
    def __init__(self):
        torch.nn.Module.__init__(self)


def _layer():
    return _Lin()


def test_from_config_round_trip():
    raw = {"quant_method": "dbf", "quantization_bits": [{"self_attn.q_proj": {"bits": 1.5, "method": "dbf"},
                                                         "mlp.down_proj": {"bits": 1.0, "method": "dbf"}}]}
    cfg = D.DbfConfig.from_config(raw)
    assert cfg.get_name() == "dbf" and cfg.quantization_bits == raw["quantization_bits"]


def test_get_quant_method_attaches_module_config():
    cfg = D.DbfConfig.from_config({"quantization_bits": [{"self_attn.q_proj": {"bits": 1.5, "method": "dbf"}}]})
    layer = _layer()
    m = cfg.get_quant_method(layer, "model.layers.0.self_attn.q_proj")
    assert isinstance(m, D.DBFLinearMethod)
    assert layer._dbf_prefix == "model.layers.0.self_attn.q_proj"
    assert layer._dbf_mod_cfg == {"bits": 1.5, "method": "dbf"}


def test_bits_zero_and_other_method_are_unquantized():
    cfg = D.DbfConfig.from_config({"quantization_bits": [{"self_attn.q_proj": {"bits": 0, "method": "dbf"},
                                                          "mlp.up_proj": {"bits": 1, "method": "onebit"}}]})
    assert isinstance(cfg.get_quant_method(_layer(), "model.layers.0.self_attn.q_proj"), UnquantizedLinearMethod)
    assert isinstance(cfg.get_quant_method(_layer(), "model.layers.0.mlp.up_proj"), UnquantizedLinearMethod)
    assert cfg.get_quant_method(torch.nn.ReLU(), "model.layers.0.mlp.up_proj") is None


def test_rank_matches_oracle():
    for k, n, b in [(4096, 14336, 1.0), (14336, 4096, 1.0), (4096, 4096, 1.5), (64, 48, 8.0)]:
        assert D.compute_mid_features(b, k, n) == od.mid_features(b, k, n)
    assert D.compute_mid_features(1.0, 4096, 14336) == 3185


def test_create_weights_fused_layout_and_loaders():
    layer = _layer()
    layer._dbf_mod_cfg = {"bits": 1.0, "method": "dbf"}
    method = D.DBFLinearMethod(None)
    parts = [64, 32, 32]
    method.create_weights(layer, 96, parts, 96, 128, torch.float16)
    lay = od.part_layout(1.0, 96, parts)
    meta = layer._dbf_meta
    for key in ("mid_sizes", "bp1_sizes", "bp3_sizes", "bp1_offsets", "bp3_offsets",
                "scaling2_offsets", "scaling4_offsets"):
        assert meta[key] == lay[key], key
    assert layer.scaling0.shape == (3, 96)
    assert layer.bp1.numel() == sum(lay["bp1_sizes"]) and layer.bp1.dtype == torch.uint8
    for i, sid in enumerate("qkv"):
        b = torch.full((lay["bp3_sizes"][i],), i + 1, dtype=torch.uint8)
        layer.bp3.weight_loader(layer.bp3, b, sid)
        layer.scaling0.weight_loader(layer.scaling0, torch.full((96,), float(i)), sid)
    for i in range(3):
        o, s = lay["bp3_offsets"][i], lay["bp3_sizes"][i]
        assert torch.all(layer.bp3.data[o:o + s] == i + 1)
        assert torch.all(layer.scaling0.data[i] == i)
    with pytest.raises(ValueError, match="shard_id"):
        layer.bp1.weight_loader(layer.bp1, torch.zeros(lay["bp1_sizes"][0], dtype=torch.uint8))


def test_apply_without_meta_raises():
    with pytest.raises(RuntimeError, match="DBF meta not initialized"):
        D.DBFLinearMethod(None).apply(torch.nn.Module(), torch.zeros(1, 8))
