"""GPU parity of fused GPTQ modules whose parts differ in bits / group size / act-order
(oc_gptq_gemm_grouped) against the oracle, part by part."""

import numpy as np
import pytest
import torch

from oracle import gptq as og
from onecompression_amd import ops, synth

pytestmark = pytest.mark.gpu


def _np(t):
    return t.detach().cpu().numpy()


def _oracle_w(c, dtype):
    g = _np(c.g_idx) if c.g_idx is not None else og.default_g_idx(c.in_features, c.group_size)
    return og.dequantize(_np(c.qweight), _np(c.qzeros), _np(c.scales), g, c.bits, "gptq", dtype)


def _rel(y, ref):
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


# (bits, N, group size, act-order) per part
QKV_MIXED = [(4, 256, 128, False), (8, 64, 128, False), (8, 64, 128, False)]   # config-1 style q@4b, k/v@8b
ALL_BITS = [(2, 96, 128, False), (3, 64, 128, True), (4, 128, 256, False), (8, 32, -1, False)]
ODD_GROUPS = [(4, 128, 64, False), (8, 64, 128, False)]  # a group of 64: parts one after the other
# half-width parts (two n-tiles per workgroup at M <= 2) with odd n-tile counts: the last
# workgroup's second n-tile is past the part
HALF_ODD = [(4, 272, 128, False), (8, 48, 128, False), (2, 208, 128, False)]


@pytest.mark.parametrize("parts", [QKV_MIXED, ALL_BITS, ODD_GROUPS, HALF_ODD],
                         ids=["qkv", "all_bits", "odd_groups", "half_odd"])
@pytest.mark.parametrize("m", [1, 3, 16, 40])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_grouped_matches_oracle_per_part(dev, parts, m, dtype):
    k = 512
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    cases = [synth.gptq_case(f"p{i}", k, n, b, gs, act, seed=11 * i + b) for i, (b, n, gs, act) in enumerate(parts)]
    preps = []
    for c in cases:
        cd = c.to(dev)
        preps.append(ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, cd.g_idx, c.bits, c.group_size))
    x = synth.activations(m, k, td, seed=5)
    biases = [(torch.randn(c.out_features, generator=torch.Generator().manual_seed(i)) * 0.1).to(td)
              for i, c in enumerate(cases)]
    biases[1] = None  # a part without bias
    y = ops.gptq_gemm_grouped(x.to(dev), preps, [None if b is None else b.to(dev) for b in biases])
    got = _np(y.float())
    assert got.shape == (m, sum(c.out_features for c in cases))
    xb = _np(x.view(torch.int16)).view(np.uint16) if dtype == "bf16" else _np(x)
    off = 0
    for c, b in zip(cases, biases):
        bb = None if b is None else (_np(b.view(torch.int16)).view(np.uint16) if dtype == "bf16" else _np(b))
        ref = og.linear_ref(xb, _oracle_w(c, dtype), dtype, bb)
        r = _rel(got[:, off:off + c.out_features], ref)
        assert r <= 1e-2, f"part {c.name} bits={c.bits}: max rel err {r:.3e}"
        off += c.out_features


def test_grouped_equals_separate_launches(dev):
    """The one-launch grouped path and oc_gptq_gemm per part give the same bits at M = 1."""
    k = 1024
    cases = [synth.gptq_case(f"p{i}", k, n, b, 128, False, seed=i) for i, (b, n) in enumerate([(4, 512), (8, 128), (8, 128)])]
    preps = []
    for c in cases:
        cd = c.to(dev)
        preps.append(ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, None, c.bits, 128))
    x = synth.activations(1, k, torch.float16, seed=9).to(dev)
    y = ops.gptq_gemm_grouped(x, preps)
    sep = torch.cat([ops.gptq_gemm(x, p) for p in preps], dim=1)
    assert torch.equal(y, sep)
