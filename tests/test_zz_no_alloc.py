"""The allocation-free entry point oc_gptq_gemm_noalloc against oc_gptq_gemm (through the C ABI).

Both run the same launch plan, so the outputs must be identical bit for bit.  Each case makes two
calls in a row on the shared per-GPU scratch array, the second with a smaller input (its work
buffer then overlaps stale contents of the first), and checks both.
"""

import pytest
import torch

from onecompression_amd import _native as N
from onecompression_amd import ops, synth

pytestmark = pytest.mark.gpu


def _prep(dev, c):
    cd = c.to(dev)
    return ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, cd.g_idx, c.bits, c.group_size)


def _both(dev, prep, m, dtype, seed, bias=None):
    x = synth.activations(m, prep.in_features, dtype, seed=seed).to(dev)
    want = ops.gptq_gemm(x, prep, bias)
    out = torch.empty_like(want)
    got = ops.gptq_gemm_noalloc(x, prep, bias, out=out)
    torch.cuda.synchronize()
    assert got.data_ptr() == out.data_ptr()
    return want, got


@pytest.mark.parametrize("case", ["act_order", "split_k_gemm", "split_k_gemv"])
def test_noalloc_matches_workspace_entry_point(dev, plan, case):
    if case == "act_order":
        # Qwen3-8B down (12288 -> 4096, 3-bit act-order): x gathered through the scratch array
        prep = _prep(dev, synth.config_cases(2)[2])
        calls = [(64, torch.float16), (16, torch.float16)]
        ws_big = N.load().oc_gptq_workspace_bytes(64, 12288, 4096, 3, 128, 1)
        assert ws_big > 0
    elif case == "split_k_gemm":
        # Qwen3-14B gate_up at M = 2048: 64 tiles cut along K, 64 MiB of fp32 partials; then a
        # smaller M on the same layer
        c = synth.config_cases(4)[2]
        prep = _prep(dev, c)
        calls = [(2048, torch.bfloat16), (600, torch.bfloat16)]
        assert "split_tiles=64" in N.describe_gptq_plan(2048, c.in_features, c.out_features, 4, 128) or \
            torch.cuda.get_device_properties(0).multi_processor_count != 256
    else:
        # the GEMV cut along K (forced): fp32 partials of every slice, then the reduction
        plan("OC_GEMV_S", 4)
        prep = _prep(dev, synth.config_cases(1)[1])  # k_proj 4096 -> 1024, 8-bit
        calls = [(7, torch.float16), (3, torch.float16)]
    for i, (m, dt) in enumerate(calls):
        b = (torch.randn(prep.out_features, generator=torch.Generator().manual_seed(i)) * 0.1).to(dt).to(dev)
        want, got = _both(dev, prep, m, dt, seed=300 + 7 * i, bias=b if i == 1 else None)
        assert torch.equal(got, want), f"{case} call {i} (M={m}) differs from oc_gptq_gemm"


def test_noalloc_rejects_calls_beyond_the_scratch_size(dev):
    """An act-order gather of M * K * 2 bytes above the array's size is refused on the host."""
    lim = N.load().oc_gptq_noalloc_scratch_bytes()
    assert lim == 64 << 20
    prep = _prep(dev, synth.config_cases(2)[2])  # K = 12288, act-order
    m = lim // (12288 * 2) + 1
    x = torch.zeros((m, 12288), dtype=torch.float16, device=dev)
    with pytest.raises(N.OCError) as e:
        ops.gptq_gemm_noalloc(x, prep)
    assert e.value.code == N.OC_ERR_WORKSPACE and "at most" in str(e.value)
