"""GPU parity of the GPTQ path against the oracle (through the C ABI)."""

import numpy as np
import pytest
import torch

from oracle import gptq as og
from onecompression_amd import ops, synth
from onecompression_amd import _native as N

pytestmark = pytest.mark.gpu

BITS = [2, 3, 4, 8]


def _np(t):
    return t.detach().cpu().numpy()


def _case(k, n, bits, gs=128, act=False, seed=0):
    return synth.gptq_case("t", k, n, bits, gs, act, seed)


def _oracle_w(c, dtype, fmt="gptq"):
    g = _np(c.g_idx) if c.g_idx is not None else og.default_g_idx(c.in_features, c.group_size)
    return og.dequantize(_np(c.qweight), _np(c.qzeros), _np(c.scales), g, c.bits, fmt, dtype)


def _rel(y, ref):
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


@pytest.mark.parametrize("bits", BITS)
def test_unpack_codes_bit_exact(dev, bits):
    c = _case(256, 96 if bits != 3 else 64, bits, seed=bits)
    got = _np(ops.gptq_unpack_codes(c.qweight.to(dev), bits))
    want = og.unpack_int_weights(_np(c.qweight), bits, (c.out_features, c.in_features))
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("fmt", [N.OC_ZERO_RAW, N.OC_ZERO_V1, N.OC_ZERO_V2])
def test_unpack_zeros_bit_exact(dev, bits, fmt):
    c = _case(256, 128, bits, seed=10 + bits)
    got = _np(ops.gptq_unpack_zeros(c.qzeros.to(dev), bits, c.out_features, fmt))
    raw = og.unpack_zeros(_np(c.qzeros), bits, c.out_features)
    want = raw if fmt == N.OC_ZERO_RAW else og.restore_zeros(raw, bits, "gptq" if fmt == 1 else "gptq_v2")
    assert np.array_equal(got, want)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs,act", [(128, False), (32, False), (-1, False), (128, True), (64, True)])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_dequant_bit_exact(dev, bits, gs, act, dtype):
    c = _case(512, 64, bits, gs, act, seed=bits * 7 + (gs % 97))
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    cd = c.to(dev)
    g = cd.g_idx
    if g is None:
        g = torch.from_numpy(og.default_g_idx(c.in_features, gs)).to(dev)
    got = ops.gptq_dequant(cd.qweight, cd.qzeros, cd.scales, g, bits, gs, N.OC_ZERO_V1, td)
    want = _oracle_w(c, dtype)
    assert np.array_equal(_np(got.view(torch.int16)).view(np.uint16), want.view(np.uint16))


def test_dequant_config0_full_size_bit_exact(dev):
    c = synth.config_cases(0)[0]
    cd = c.to(dev)
    g = torch.from_numpy(og.default_g_idx(4096, 128)).to(dev)
    got = ops.gptq_dequant(cd.qweight, cd.qzeros, cd.scales, g, 4, 128)
    assert np.array_equal(_np(got).view(np.uint16), _oracle_w(c, "fp16").view(np.uint16))


def _gemm_check(dev, c, m, dtype, bias=False, tol=None, seed=3):
    # regression bounds well under the 1e-2 contract (the kernels measure ~3e-4 in fp16): fp16
    # products are exact in fp32, the output rounds once; bf16 rounds its output at 2^-9
    if tol is None:
        tol = 2e-3 if dtype == "fp16" else 8e-3
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    cd = c.to(dev)
    prep = ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, cd.g_idx, c.bits, c.group_size)
    x = synth.activations(m, c.in_features, td, seed=seed)
    b = (torch.randn(c.out_features) * 0.1).to(td) if bias else None
    y = ops.gptq_gemm(x.to(dev), prep, None if b is None else b.to(dev))
    torch.cuda.synchronize()
    w = _oracle_w(c, dtype)
    xb = _np(x.view(torch.int16)).view(np.uint16) if dtype == "bf16" else _np(x)
    bb = None if b is None else (_np(b.view(torch.int16)).view(np.uint16) if dtype == "bf16" else _np(b))
    ref = og.linear_ref(xb, w, dtype, bb)
    got = _np(y.float())
    assert got.shape == ref.shape
    r = _rel(got, ref)
    assert r <= tol, f"max rel err {r:.3e} > {tol}"
    return r


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [1, 5, 16, 17, 40, 64])
def test_gemm_small_m(dev, bits, m):
    _gemm_check(dev, _case(1024, 256 if bits != 3 else 320, bits, seed=bits + m), m, "fp16")


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs,act", [(32, False), (64, False), (-1, False), (128, True)])
def test_gemm_groups_and_act_order(dev, bits, gs, act):
    _gemm_check(dev, _case(1024, 192, bits, gs, act, seed=bits), 3, "fp16", bias=True)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [1, 24, 100])
def test_gemm_bf16(dev, bits, m):
    _gemm_check(dev, _case(512, 128, bits, seed=40 + bits), m, "bf16", bias=True)


def test_gemm_exact_zero_probe(dev):
    """test_gptq_layer_pack.py:338-392 through the fused kernel: qweight=0,
    scale=1, one-hot x -> columns with raw zero 0 give exactly 0, others -1."""
    k = n = 128
    for bits in BITS:
        raw = np.ones((1, n), dtype=np.int32)
        raw[:, :4] = 0
        qw = torch.from_numpy(og.pack_int_weights(np.zeros((n, k), np.int32), bits)).to(dev)
        qz = torch.from_numpy(og.pack_zeros(raw - 1, bits)).to(dev)
        sc = torch.ones((1, n), dtype=torch.float16, device=dev)
        prep = ops.gptq_prepare(qw, qz, sc, None, bits, -1)
        x = torch.zeros((1, k), dtype=torch.float16, device=dev)
        x[0, 0] = 1
        y = ops.gptq_gemm(x, prep).float().cpu()[0]
        assert torch.all(y[:4] == 0) and torch.all(y[4:] == -1), bits


@pytest.mark.parametrize("idx", range(7))
def test_gemm_config1_projection_m1(dev, idx):
    c = synth.config_cases(1)[idx]
    _gemm_check(dev, c, 1, "fp16")


def test_gemm_config2_act_order_m16(dev):
    c = synth.config_cases(2)[2]  # down 12288 -> 4096, 3-bit, act-order
    _gemm_check(dev, c, 16, "fp16")


def test_gemm_repeatable_split_k(dev, plan):
    """The split-K path (forced) is deterministic and matches the unsplit one."""
    c = synth.config_cases(1)[1].to(dev)  # k_proj 4096 -> 1024
    prep = ops.gptq_prepare(c.qweight, c.qzeros, c.scales, None, c.bits, 128)
    x = synth.activations(3, 4096).to(dev)
    y1 = ops.gptq_gemm(x, prep).clone()
    plan("OC_GEMV_S", "4")
    y4 = ops.gptq_gemm(x, prep)
    for _ in range(3):
        assert torch.equal(ops.gptq_gemm(x, prep), y4)
    torch.cuda.synchronize()
    assert float((y4.float() - y1.float()).abs().max()) <= 1e-2 * float(y1.float().abs().max())


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("w,nt", [(4, 1), (8, 1), (16, 1), (4, 2), (8, 2), (16, 2)])
def test_gemv_plan_variants(dev, plan, bits, w, nt):
    """Every GEMV launch shape (waves per workgroup x n-tiles per wave), with
    several k-units per wave, M = 1 and M = 7 (x rows bounced through LDS by a
    subset of lanes)."""
    plan("OC_GEMV_W", str(w))
    plan("OC_GEMV_NT", str(nt))
    c = _case(4096, 256 if bits != 3 else 320, bits, seed=60 + bits)
    for m in (1, 7):
        _gemm_check(dev, c, m, "fp16", bias=m == 7)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [17, 32, 48, 64, 65, 100, 128, 130, 200])
def test_gemm_mid_m(dev, bits, m, plan):
    """16 < M < 256 on the tiled GEMM (tile height 64, 128 or 256 by M), with bias on even M."""
    plan("OC_GEMM_MIN_M", "17")
    _gemm_check(dev, _case(2048, 320 if bits == 3 else 256, bits, seed=70 + bits + m), m, "fp16", bias=m % 2 == 0)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("mt", ["1", "2", "4"])
def test_gemm_tile_heights(dev, plan, bits, mt):
    """Every tile height at M below, at and above it; K = 4096 on 256 columns splits the few
    tiles along K (fp32 partials, fixup kernel)."""
    plan("OC_GEMM_MIN_M", "17")
    plan("OC_GEMM_MT", mt)
    c = _case(4096, 320 if bits == 3 else 256, bits, seed=80 + bits)
    for m in (24, 96, 160):
        _gemm_check(dev, c, m, "fp16" if m != 96 else "bf16", bias=m == 96)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("gs,act,dtype,k", [(64, False, "fp16", 1024), (32, False, "bf16", 1056),
                                            (128, True, "bf16", 2048), (-1, False, "fp16", 1056)])
def test_gemm_mid_groups(dev, plan, bits, gs, act, dtype, k):
    """Tiled GEMM at mid M with groups of 32/64 (256-row tiles), act-order, one group and K not
    a multiple of the k-unit."""
    plan("OC_GEMM_MIN_M", "17")
    c = _case(k, 320 if bits == 3 else 272, bits, gs, act, seed=90 + bits)
    for m in (40, 128):
        _gemm_check(dev, c, m, dtype, bias=m == 40)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m,k,n,gs,act,dtype", [
    (128, 1024, 256, 128, False, "fp16"),
    (300, 1056, 272, 32, False, "bf16"),     # ragged M, K not a multiple of the k-unit, N not of 256
    (256, 2048, 512, 128, True, "fp16"),     # act-order
    (129, 512, 528, -1, False, "bf16"),      # one group, bias below
])
def test_gemm_large_m(dev, bits, m, k, n, gs, act, dtype):
    if bits == 3 and n % 32:
        n = (n + 31) // 32 * 32
    c = _case(k, n, bits, gs, act, seed=bits * 31 + m)
    _gemm_check(dev, c, m, dtype, bias=(m == 129))


def test_gemm_large_m_config4_shape(dev):
    c = synth.gptq_case("o", 5120, 5120, 4, 128, False, seed=3)
    _gemm_check(dev, c, 512, "bf16")


@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_gemm_split_tail(dev, plan, dtype):
    """260 tiles of 256 x 256 on a 256-CU part: 256 whole tiles plus 4 tiles cut
    along K whose fp32 partials k_gemm_fixup sums (with bias).  The split result
    matches the unsplit launch and, on the tail tiles' columns, the oracle."""
    k, n, m = 1024, 66560, 130
    c = synth.gptq_case("t", k, n, 4, 128, False, seed=91)
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    cd = c.to(dev)
    prep = ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, None, 4, 128)
    x = synth.activations(m, k, td, seed=5).to(dev)
    b = (torch.randn(n) * 0.1).to(td).to(dev)
    y = ops.gptq_gemm(x, prep, b)
    assert torch.equal(ops.gptq_gemm(x, prep, b), y)  # deterministic split order
    plan("OC_GEMM_SPLIT", "1")
    y1 = ops.gptq_gemm(x, prep, b)
    torch.cuda.synchronize()
    ref_scale = float(y1.float().abs().max())
    assert float((y.float() - y1.float()).abs().max()) <= 1e-2 * ref_scale
    n0, n1 = 65536 - 256, n  # last whole tile and the 4 split tiles
    sub = synth.GPTQCase("t", k, n1 - n0, 4, 128, False, c.qweight[:, n0:n1].contiguous(),
                         c.qzeros[:, n0 // 8:n1 // 8].contiguous(), c.scales[:, n0:n1].contiguous(), None)
    w = _oracle_w(sub, dtype)
    xb = _np(x.cpu().view(torch.int16)).view(np.uint16) if dtype == "bf16" else _np(x.cpu())
    bs = b[n0:n1].cpu()
    bb = _np(bs.view(torch.int16)).view(np.uint16) if dtype == "bf16" else _np(bs)
    ref = og.linear_ref(xb, w, dtype, bb)
    r = _rel(_np(y[:, n0:n1].float()), ref)
    assert r <= 1e-2, f"max rel err {r:.3e}"


# Wide layers at M <= 8 take the streaming GEMV (one wave per n-tile, x staged in LDS):
# every bit width, partial last workgroup (N not a multiple of 64 columns), bias, act-order, bf16.
@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [1, 2, 3, 8])
def test_gemm_streaming_wide(dev, bits, m):
    n = 16384 + 48 if bits != 3 else 16384 + 32  # >= 1024 n-tiles, last workgroup partial
    _gemm_check(dev, _case(512, n, bits, seed=60 + bits + m), m, "fp16", bias=(m == 3))


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("case", ["act", "bf16", "g256", "narrow_forced"])
def test_gemm_streaming_variants(dev, bits, case, plan):
    if case == "act":
        _gemm_check(dev, _case(1024, 16384, bits, 128, True, seed=70 + bits), 2, "fp16", bias=True)
    elif case == "bf16":
        _gemm_check(dev, _case(512, 16384, bits, seed=80 + bits), 4, "bf16", bias=True)
    elif case == "g256":
        _gemm_check(dev, _case(1024, 16384, bits, 256, False, seed=90 + bits), 1, "fp16")
    else:  # forced on a narrow layer: fewer n-tiles than one workgroup's 4 waves in the last group
        plan("OC_GEMV_STREAM", "1")
        _gemm_check(dev, _case(768, 80 if bits != 3 else 96, bits, seed=95 + bits), 5, "fp16", bias=True)


# Layers whose n-tiles do not give every CU the same number of 4-wave workgroups take the
# balanced streaming GEMV (8 waves share T n-tiles' units evenly, so a wave's range may start or
# end inside an n-tile; the partial sums of an n-tile meet in LDS).  On 256 CUs these n give
# T = 1..8 n-tiles per workgroup, a partial last workgroup, and (T = 1 with two units per n-tile)
# waves with no units at all.
BAL_SHAPES = [(4096, 28672, 1), (512, 16384 + 32, 3), (1024, 2048 + 32, 4), (512, 1024, 2),
              (1024, 4096 + 96, 1), (640, 28672 + 32, 2), (256, 9600, 4), (768, 14400, 1),
              (1152, 22400, 3)]


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("k,n,m", BAL_SHAPES)
def test_gemm_streaming_balanced(dev, bits, k, n, m, plan):
    plan("OC_GEMV_STREAM", "1")
    plan("OC_GEMV_STREAM_BAL", "1")
    _gemm_check(dev, _case(k, n, bits, seed=500 + bits + m), m, "fp16", bias=(m != 1))


def test_config1_merged_gate_up_m1_to_m4(dev):
    """Config 1's merged gate|up layer (4096 -> 28672, 3-bit) at its real shape: k_gemv_stream at
    M = 1, 2 and the balanced kernel at M = 3, 4, all against one oracle dequantization."""
    gu = synth.layer_calls(1)[2][0]
    cd = gu.to(dev)
    prep = ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, None, gu.bits, gu.group_size)
    w = _oracle_w(gu, "fp16")
    for m in (1, 2, 3, 4):
        x = synth.activations(m, gu.in_features, torch.float16, seed=600 + m)
        y = ops.gptq_gemm(x.to(dev), prep)
        ref = og.linear_ref(_np(x), w, "fp16", None)
        r = _rel(_np(y.float()), ref)
        assert r <= 1e-2, f"M={m}: max rel err {r:.3e}"


# K = 8192 at M = 4: x and its k-block sums take 70 KB of LDS (86 KB with the balanced kernel's
# partial sums), above the 64 KB of earlier CDNA parts.
@pytest.mark.parametrize("bal", ["0", "1"])
def test_gemm_streaming_large_lds(dev, bal, plan):
    plan("OC_GEMV_STREAM_BAL", bal)
    _gemm_check(dev, _case(8192, 16384 + 32, 4, seed=540), 4, "fp16", bias=True)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("case", ["act", "bf16", "g256"])
def test_gemm_streaming_balanced_variants(dev, bits, case, plan):
    plan("OC_GEMV_STREAM_BAL", "1")
    if case == "act":
        _gemm_check(dev, _case(1024, 17408, bits, 128, True, seed=510 + bits), 2, "fp16", bias=True)
    elif case == "bf16":
        _gemm_check(dev, _case(512, 17408, bits, seed=520 + bits), 4, "bf16", bias=True)
    else:
        _gemm_check(dev, _case(1024, 17408, bits, 256, False, seed=530 + bits), 1, "fp16")


# The streaming GEMV folds the zero point in through per-k-block sums of x (an fp32 offset term
# of 1024 sum(x) that cancels): tiny activations and a wide dynamic range stay within the bar.
@pytest.mark.parametrize("m", [1, 4])
@pytest.mark.parametrize("scale", ["tiny", "wide"])
def test_gemm_streaming_3bit_small_and_wide_x(dev, m, scale):
    c = _case(1024, 16384, 3, seed=170 + m)
    cd = c.to(dev)
    prep = ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, None, 3, 128)
    g = torch.Generator().manual_seed(171 + m)
    x = torch.randn((m, 1024), generator=g)
    x = x * 1e-3 if scale == "tiny" else x * torch.pow(10.0, torch.empty((m, 1024)).uniform_(-4, 2, generator=g))
    x = x.to(torch.float16)
    y = ops.gptq_gemm(x.to(dev), prep)
    ref = og.linear_ref(_np(x), _oracle_w(c, "fp16"), "fp16", None)
    r = _rel(_np(y.float()), ref)
    assert r <= 1e-2, f"max rel err {r:.3e}"


# Wide layers at mid M take the streaming GEMM (k-block x staging ring, MB row blocks per B
# operand); K = 14336 at M = 4 takes it too (x does not fit the GEMV stream's LDS).
@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [9, 16, 17, 32])
def test_gemm_streaming_mid_m(dev, bits, m):
    n = 16384 + 48 if bits != 3 else 16384 + 32
    _gemm_check(dev, _case(1024, n, bits, seed=120 + bits + m), m, "fp16", bias=(m == 17))


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("case", ["act", "bf16", "g256", "long_k_m4", "narrow_forced"])
def test_gemm_streaming_mid_m_variants(dev, bits, case, plan):
    if case == "act":
        _gemm_check(dev, _case(1024, 16384, bits, 128, True, seed=130 + bits), 20, "fp16", bias=True)
    elif case == "bf16":
        _gemm_check(dev, _case(1024, 16384, bits, seed=140 + bits), 24, "bf16", bias=True)
    elif case == "g256":
        _gemm_check(dev, _case(1024, 16384, bits, 256, False, seed=150 + bits), 12, "fp16")
    elif case == "long_k_m4":
        _gemm_check(dev, _case(14336, 16384, bits, seed=155 + bits), 4, "fp16")
    else:
        plan("OC_GEMM_STREAM", "1")
        _gemm_check(dev, _case(768, 80 if bits != 3 else 96, bits, seed=160 + bits), 30, "fp16", bias=True)


# The streaming GEMM at 32 < M <= 128 (4 or 8 row blocks per B operand, dequantised B operand) and
# its K split across workgroups (fp32 partials summed by k_splitk_reduce), forced by plan knobs:
# splits the planner reduces to an even unit count, a ragged last n-tile, bias, bf16, act-order and
# groups of 256.  ntw = 2: two n-tiles per wave (45 or 46 n-tiles: the last wave's second n-tile
# lies past the end).  Tolerances are regression bounds well under the 1e-2 contract.
@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [33, 64, 100, 128])
@pytest.mark.parametrize("split", [1, 2, 4])
@pytest.mark.parametrize("ntw", [1, 2])
def test_gemm_stream_mid_m_split(dev, bits, m, split, ntw, plan):
    plan("OC_GEMM_STREAM", 1)
    plan("OC_GEMM_STREAM_S", split)
    plan("OC_GEMM_STREAM_NTW", ntw)
    n = 720 if bits != 3 else 736
    _gemm_check(dev, _case(2048, n, bits, seed=400 + 7 * bits + m + split), m, "fp16", bias=(split == 2), tol=2e-3)


# Rows split across workgroups as well (grid.z = 64-row halves, each with its own x slice, output
# rows and partial rows), with and without K splits; a ragged second half.
@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [65, 100, 128])
@pytest.mark.parametrize("split", [1, 2, 4])
def test_gemm_stream_row_split(dev, bits, m, split, plan):
    plan("OC_GEMM_STREAM", 1)
    plan("OC_GEMM_STREAM_MZ", 2)
    plan("OC_GEMM_STREAM_S", split)
    n = 720 if bits != 3 else 736
    _gemm_check(dev, _case(2048, n, bits, seed=470 + 7 * bits + m + split), m, "fp16", bias=(split == 1), tol=2e-3)


# The tiled GEMM at the mid M the streaming GEMM now serves (64-row tiles, K split pieces).
@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("m", [33, 64, 100])
def test_gemm_tiled_mid_m(dev, bits, m, plan):
    plan("OC_GEMM_STREAM", 0)
    _gemm_check(dev, _case(2048, 720 if bits != 3 else 736, bits, seed=460 + bits + m), m, "fp16", bias=True,
                tol=2e-3)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("case", ["bf16", "act", "g256", "wide"])
@pytest.mark.parametrize("ntw", [1, 2])
def test_gemm_stream_mid_m_variants(dev, bits, case, ntw, plan):
    plan("OC_GEMM_STREAM", 1)
    plan("OC_GEMM_STREAM_NTW", ntw)
    if case == "bf16":
        plan("OC_GEMM_STREAM_S", 2)
        _gemm_check(dev, _case(2048, 512, bits, seed=420 + bits), 96, "bf16", bias=True, tol=8e-3)
    elif case == "act":
        plan("OC_GEMM_STREAM_S", 4)
        _gemm_check(dev, _case(4096, 512, bits, 128, True, seed=430 + bits), 72, "fp16", bias=True, tol=2e-3)
    elif case == "g256":
        plan("OC_GEMM_STREAM_S", 2)
        _gemm_check(dev, _case(4096, 400 if bits != 3 else 416, bits, 256, False, seed=440 + bits), 50, "fp16",
                    tol=2e-3)
    else:
        _gemm_check(dev, _case(1024, 16384, bits, seed=450 + bits), 120, "fp16", tol=2e-3)


# The large-M GEMM with K not a multiple of 128: the last k-block's x chunks past K load as zeros
# through the buffer range check (the padded codes dequantise to -z s, so stale x there would show).
@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("k", [160, 288, 800])
def test_gemm_large_m_k_tail(dev, bits, k):
    _gemm_check(dev, _case(k, 512, bits, 32 if k % 64 else 64, seed=180 + bits + k), 300, "fp16")
