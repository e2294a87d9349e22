"""GPU parity of the DBF / MDBF sign path against the oracle (through the C ABI)."""

import numpy as np
import pytest
import torch

from oracle import dbf as od
from oracle import gptq as og
from onecompression_amd import dbf as D
from onecompression_amd import dbf_ops
from onecompression_amd.vllm_compat import HAS_VLLM, LinearBase

pytestmark = pytest.mark.gpu


def _t(a, dev):
    return torch.from_numpy(np.ascontiguousarray(a)).to(dev)


def _rel(y, ref):
    return float(np.max(np.abs(y - ref)) / max(np.max(np.abs(ref)), 1e-30))


def _factors(k, n, seed, bits=1.0):
    rng = np.random.default_rng(seed)
    r = od.mid_features(bits, k, n)
    bp1 = od.pack_binary(rng.choice([-1, 1], size=(r, k)))
    bp3 = od.pack_binary(rng.choice([-1, 1], size=(n, r)))
    s0, s2, s4 = [(np.abs(rng.normal(0, 0.05, d)) + 1e-3).astype(np.float16) for d in (k, r, n)]
    return r, bp1, bp3, s0, s2, s4


def test_unpack_known_answers(dev):
    got = dbf_ops.unpack_signs(_t(np.array([0b11001100, 0b00110011], np.uint8), dev), 2, 8).cpu().numpy()
    assert got.tolist() == [[1, 1, -1, -1, 1, 1, -1, -1], [-1, -1, 1, 1, -1, -1, 1, 1]]
    got = dbf_ops.unpack_signs(_t(np.array([0b10101010], np.uint8), dev), 1, 8).cpu().numpy()
    assert got.tolist() == [[1, -1, 1, -1, 1, -1, 1, -1]]


@pytest.mark.parametrize("shape", [(5, 7), (13, 11), (3185, 64), (40, 3185)])
def test_unpack_bit_exact(dev, shape):
    rng = np.random.default_rng(shape[0])
    m = rng.choice([-1, 1], size=shape).astype(np.int8)
    p = od.pack_binary(m)
    got = dbf_ops.unpack_signs(_t(p, dev), *shape).cpu().numpy()
    assert np.array_equal(got, m) and np.array_equal(got, od.unpack_binary_factor(p, shape))


def test_sign_matmul_known_answer(dev):
    """test_dbf_naive.py:110-151 through the kernel: [[-4, 4], [4, -4]]."""
    f = dbf_ops.sign_prepare(_t(np.array([0b10101010, 0b01010101], np.uint8), dev), 2, 8)
    x = torch.tensor([[1, 2, 3, 4, 5, 6, 7, 8], [8, 7, 6, 5, 4, 3, 2, 1]], dtype=torch.float16, device=dev)
    out = torch.empty((2, 8), dtype=torch.float16, device=dev)
    dbf_ops.sign_gemm([(f, x, None, None)], 2, 2, torch.float16, out, 8)
    assert out[:, :2].float().cpu().tolist() == [[-4, 4], [4, -4]]


@pytest.mark.parametrize("k,n,m", [(256, 192, 1), (256, 192, 3), (640, 256, 16), (512, 384, 37),
                                   (4096, 14336, 1), (14336, 4096, 1), (4096, 14336, 32),
                                   # M >= 128: the large-M GEMM core with the sign decoder
                                   (512, 384, 130), (640, 1000, 300), (4096, 14336, 160)])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_dbf_forward(dev, k, n, m, dtype):
    r, bp1, bp3, s0, s2, s4 = _factors(k, n, k + n + m)
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(td)
    prep = dbf_ops.dbf_prepare(_t(s0, dev), _t(bp1, dev), _t(s2, dev), _t(bp3, dev), _t(s4, dev), k, r, n)
    y = dbf_ops.dbf_forward(x.to(dev), [prep]).float().cpu().numpy()
    if dtype == "bf16":  # the reference casts the fp16 scalings to x.dtype (vllm_plugin.py:286-292)
        xn = x.view(torch.int16).numpy().view(np.uint16)
        sc = [og.f32_to_bf16_bits(v.astype(np.float32)) for v in (s0, s2, s4)]
    else:
        xn, sc = x.numpy(), [s0, s2, s4]
    ref = od.dbf_forward(xn, sc[0], bp1, sc[1], bp3, sc[2], k, r, n, dtype=dtype)
    tol = 1e-2 if dtype == "fp16" else 2e-2
    assert _rel(y, ref) <= tol, _rel(y, ref)


def test_dbf_all_plus_signs_fused_parts(dev):
    """test_dbf_gemlite_fallback.py:274-329 through the kernels: all signs +1,
    distinct per-part scalings, three fused parts; allclose(atol=rtol=1e-2)."""
    k, mid, n_out, parts, batch = 64, 32, 48, 3, 4
    s0 = torch.stack([torch.linspace(0.5, 1.5, k, dtype=torch.float16) * (1.0 + 0.1 * p) for p in range(parts)])
    s2 = torch.linspace(0.5, 1.5, mid * parts, dtype=torch.float16)
    s4 = torch.linspace(0.5, 1.5, n_out * parts, dtype=torch.float16)
    bp1 = torch.full(((mid * k + 7) // 8,), 0xFF, dtype=torch.uint8)
    bp3 = torch.full(((n_out * mid + 7) // 8,), 0xFF, dtype=torch.uint8)
    preps = [dbf_ops.dbf_prepare(s0[p].to(dev), bp1.to(dev), s2[p * mid:(p + 1) * mid].to(dev), bp3.to(dev),
                                 s4[p * n_out:(p + 1) * n_out].to(dev), k, mid, n_out) for p in range(parts)]
    x = torch.randn(batch, k, generator=torch.Generator().manual_seed(0))
    y = dbf_ops.dbf_forward(x.half().to(dev), preps).float().cpu()
    exp = []
    for p in range(parts):
        h = (x.half().float() * s0[p].float()) @ torch.ones(mid, k).t()
        h = h * s2[p * mid:(p + 1) * mid].float()
        exp.append((h @ torch.ones(n_out, mid).t()) * s4[p * n_out:(p + 1) * n_out].float())
    exp = torch.cat(exp, dim=-1)
    assert y.shape == (batch, n_out * parts)
    assert torch.allclose(y, exp, atol=1e-2, rtol=1e-2)


@pytest.mark.skipif(HAS_VLLM, reason="layer built with the local LinearBase stand-in")
def test_dbf_plugin_layer_fused_qkv(dev):
    qb = [{f"self_attn.{p}_proj": {"bits": 1.0, "method": "dbf"} for p in "qkv"}]
    cfg = D.DbfConfig.from_config({"quantization_bits": qb})
    k, parts = 256, [256, 64, 64]
    layer = LinearBase(k, sum(parts), bias=True, quant_config=cfg, prefix="model.layers.0.self_attn.qkv_proj",
                       output_partition_sizes=parts)
    ref_parts, rng = [], np.random.default_rng(1)
    for i, (sid, n) in enumerate(zip("qkv", parts)):
        r, bp1, bp3, s0, s2, s4 = _factors(k, n, 10 + i)
        assert r == layer._dbf_meta["mid_sizes"][i]
        for name, val in (("scaling0", s0), ("scaling2", s2), ("scaling4", s4), ("bp1", bp1), ("bp3", bp3)):
            p = getattr(layer, name)
            p.weight_loader(p, torch.from_numpy(val), sid)
        ref_parts.append((r, bp1, bp3, s0, s2, s4, n))
    bias = rng.normal(0, 0.01, sum(parts)).astype(np.float16)
    layer.bias.data.copy_(torch.from_numpy(bias))
    layer.to(dev)
    layer.quant_method.process_weights_after_loading(layer)
    x = torch.randn(3, k, generator=torch.Generator().manual_seed(2)).half()
    y = layer(x.to(dev)).float().cpu().numpy()
    ref = np.concatenate([od.dbf_forward(x.numpy(), s0, bp1, s2, bp3, s4, k, r, n)
                          for (r, bp1, bp3, s0, s2, s4, n) in ref_parts], axis=1) + bias.astype(np.float32)
    assert _rel(y, ref) <= 1e-2


def _mdbf_path(n, m, r, l, seed):
    rng = np.random.default_rng(seed)
    amp = lambda *s: (np.abs(rng.normal(0, 0.3, s)) + 1e-2).astype(np.float16)  # noqa: E731
    return dict(A_sign_packed=od.pack_binary(rng.choice([-1, 1], size=(n, r))), A_shape=(n, r),
                B_sign_packed=od.pack_binary(rng.choice([-1, 1], size=(r, m))), B_shape=(r, m),
                A_amp=amp(n, l), B_amp=amp(m, l), Q_U_amp=amp(r, l), Q_V_amp=amp(r, l))


@pytest.mark.parametrize("P,l,m_rows", [(2, 1, 1), (2, 1, 32), (1, 2, 4), (2, 2, 1), (2, 2, 16),
                                        (2, 1, 200), (1, 2, 150), (2, 2, 140)])  # M > 16: partial slots
def test_mdbf_forward(dev, P, l, m_rows):
    n, m = 384, 256
    r = od.mid_features(1.0, m, n)
    paths = [_mdbf_path(n, m, r, l, 100 * P + 10 * l + i) for i in range(P)]
    preps = [dbf_ops.mdbf_prepare_path(_t(p["A_sign_packed"], dev), p["A_shape"], _t(p["B_sign_packed"], dev),
                                       p["B_shape"], _t(p["A_amp"], dev), _t(p["B_amp"], dev),
                                       _t(p["Q_U_amp"], dev), _t(p["Q_V_amp"], dev)) for p in paths]
    x = torch.randn(m_rows, m, generator=torch.Generator().manual_seed(3)).half()
    y = dbf_ops.mdbf_forward(x.to(dev), preps).float().cpu().numpy()
    ref = od.mdbf_forward(x.numpy(), paths)
    assert _rel(y, ref) <= 1e-2, _rel(y, ref)


@pytest.mark.parametrize("m", [1, 5, 16, 40, 140])  # GEMV (M <= 16) and the GEMM core (tile heights 64..256)
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
def test_sign_gemm_fill_and_bias(dev, dtype, m):
    """Sign matmul: pre/post scales, bias, zero columns R..fill_to, ld_out > fill_to."""
    kd, R, fill_to, ld_out = 300, 37, 40, 48
    rng = np.random.default_rng(7)
    signs = rng.choice([-1, 1], size=(R, kd))
    f = dbf_ops.sign_prepare(_t(od.pack_binary(signs), dev), R, kd)
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    x = torch.zeros((m, 304), dtype=td)
    x[:, :kd] = torch.randn(m, kd, generator=torch.Generator().manual_seed(1)).to(td)
    pre = torch.zeros(304, dtype=td)
    pre[:kd] = torch.rand(kd, generator=torch.Generator().manual_seed(2)).to(td) + 0.5
    post = (torch.rand(R, generator=torch.Generator().manual_seed(3)) + 0.5).to(td)
    bias = (torch.randn(R, generator=torch.Generator().manual_seed(4)) * 0.1).to(td)
    out = torch.full((m, ld_out), 7.0, dtype=td, device=dev)
    dbf_ops.sign_gemm([(f, x.to(dev), pre.to(dev), post.to(dev))], m, R, td, out, ld_out, fill_to=fill_to,
                      bias=bias.to(dev))
    o = out.float().cpu()
    xs = (x[:, :kd].float() * pre[:kd].float()).to(td).float()  # RNE(x * pre) as the reference
    ref = (xs @ torch.from_numpy(signs).float().t()) * post.float() + bias.float()
    assert _rel(o[:, :R].numpy(), ref.numpy()) <= 1e-2
    assert torch.all(o[:, R:fill_to] == 0)
    assert torch.all(o[:, fill_to:] == 7.0)


# 13 <= M <= 64 on the streaming sign kernel (x staged per k-block with the pre scale applied,
# two k-blocks per step up to 32 rows — an odd k-block count leaves the last step half past the
# split — K split over workgroups with an ordered reduce) and, pinned, on the large-M GEMM core
# (64-row tiles, K split with fp32 partials and a fixup): pre and post scales, bias, fill_to of the
# rank stage, a rank stage of one-k-block units, bf16, row counts at and past each row-block size.
@pytest.mark.parametrize("m", [13, 16, 17, 32, 33, 48, 63, 64])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("path", ["stream", "gemm", "stream_s1", "stream_s3", "stream_mz2"])
def test_dbf_mid_m(dev, m, dtype, path, plan):
    if path == "gemm":
        plan("OC_SIGN_STREAM", 0)
    elif path == "stream_mz2":  # rows split across workgroups as well (two row blocks)
        plan("OC_SIGN_STREAM_MZ", 2)
    elif path != "stream":
        plan("OC_SIGN_STREAM_S", int(path[-1]))
    k, n = 1408, 720  # r = 476: rank stage 30 tiles x 11 k-blocks, output stage 45 tiles x 4 k-blocks
    r, bp1, bp3, s0, s2, s4 = _factors(k, n, 900 + m)
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).to(td)
    prep = dbf_ops.dbf_prepare(_t(s0, dev), _t(bp1, dev), _t(s2, dev), _t(bp3, dev), _t(s4, dev), k, r, n)
    bias = (torch.randn(n, generator=torch.Generator().manual_seed(5)) * 0.05).to(td)
    y = dbf_ops.dbf_forward(x.to(dev), [prep], bias=bias.to(dev)).float().cpu().numpy()
    if dtype == "bf16":
        xn = x.view(torch.int16).numpy().view(np.uint16)
        sc = [og.f32_to_bf16_bits(v.astype(np.float32)) for v in (s0, s2, s4)]
        bn = bias.view(torch.int16).numpy().view(np.uint16)
    else:
        xn, sc, bn = x.numpy(), [s0, s2, s4], bias.numpy()
    ref = od.dbf_forward(xn, sc[0], bp1, sc[1], bp3, sc[2], k, r, n, dtype=dtype, bias=bn)
    assert _rel(y, ref) <= (2e-3 if dtype == "fp16" else 8e-3), _rel(y, ref)


@pytest.mark.parametrize("m", [24, 32])
def test_mdbf_mid_m_two_paths(dev, m):
    n, mm = 400, 272
    r = od.mid_features(1.0, mm, n)
    paths = [_mdbf_path(n, mm, r, 1, 700 + i) for i in range(2)]
    preps = [dbf_ops.mdbf_prepare_path(_t(p["A_sign_packed"], dev), p["A_shape"], _t(p["B_sign_packed"], dev),
                                       p["B_shape"], _t(p["A_amp"], dev), _t(p["B_amp"], dev),
                                       _t(p["Q_U_amp"], dev), _t(p["Q_V_amp"], dev)) for p in paths]
    x = torch.randn(m, mm, generator=torch.Generator().manual_seed(9)).half()
    y = dbf_ops.mdbf_forward(x.to(dev), preps).float().cpu().numpy()
    ref = od.mdbf_forward(x.numpy(), paths)
    assert _rel(y, ref) <= 2e-3, _rel(y, ref)


# Several terms summed into one output, signed per-column post scales (+1 without a post vector).
# The large-M sign GEMM (m = 140, and path "gemm") sums them in one accumulation, each term's post
# scale folded into its +-1 operand, with K-split pieces over the concatenated k-blocks; without a
# bias the zero columns R..fill_to come out of the GEMM itself.  The streaming sign kernel (m = 40:
# "auto", and "s2" with two K splits per term) runs the terms side by side, each writing its own
# post-scaled fp32 partial, which k_sign_reduce adds in term order with the bias (a call with a bias
# and zero columns takes the GEMM path).
@pytest.mark.parametrize("m,path", [(40, "auto"), (40, "gemm"), (40, "s2"), (140, "auto")])
@pytest.mark.parametrize("dtype", ["fp16", "bf16"])
@pytest.mark.parametrize("n_terms,with_bias,fill", [(1, False, True), (2, False, True), (3, False, True),
                                                    (4, True, True), (4, True, False)])
def test_sign_gemm_terms_signed_scales(dev, m, path, dtype, n_terms, with_bias, fill, plan):
    if path == "gemm":
        plan("OC_SIGN_STREAM", 0)
    elif path == "s2":
        plan("OC_SIGN_STREAM_S", 2)
    R, ld_out = 530, 544
    fill_to = 536 if fill else R
    kds = [300, 260, 330, 270][:n_terms]
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    rng = np.random.default_rng(40 + n_terms + m)
    terms, ref = [], torch.zeros(m, R)
    for i, kd in enumerate(kds):
        signs = rng.choice([-1, 1], size=(R, kd))
        f = dbf_ops.sign_prepare(_t(od.pack_binary(signs), dev), R, kd)
        ldx = (kd + 7) // 8 * 8
        x = torch.zeros((m, ldx), dtype=td)
        x[:, :kd] = torch.randn(m, kd, generator=torch.Generator().manual_seed(10 + i)).to(td)
        pre = None
        if n_terms == 3:  # the terms of one call all have a pre scale or none
            pre = torch.zeros(ldx, dtype=td)
            pre[:kd] = (torch.rand(kd, generator=torch.Generator().manual_seed(20 + i)) + 0.5).to(td)
        post = None
        if i != 2:  # term 2 has no post vector (scale 1)
            post = (torch.rand(R, generator=torch.Generator().manual_seed(30 + i)) + 0.25).to(td)
            post[torch.rand(R, generator=torch.Generator().manual_seed(50 + i)) < 0.4] *= -1
        xs = x[:, :kd].float() if pre is None else (x[:, :kd].float() * pre[:kd].float()).to(td).float()
        t = xs @ torch.from_numpy(signs).float().t()
        ref += t if post is None else t * post.float()
        terms.append((f, x.to(dev), None if pre is None else pre.to(dev), None if post is None else post.to(dev)))
    bias = None
    if with_bias:
        bias = (torch.randn(R, generator=torch.Generator().manual_seed(60)) * 0.1).to(td)
        ref += bias.float()
    out = torch.full((m, ld_out), 7.0, dtype=td, device=dev)
    dbf_ops.sign_gemm(terms, m, R, td, out, ld_out, fill_to=fill_to, bias=None if bias is None else bias.to(dev))
    o = out.float().cpu()
    r = _rel(o[:, :R].numpy(), ref.numpy())
    assert r <= (2e-3 if dtype == "fp16" else 8e-3), r
    assert torch.all(o[:, R:fill_to] == 0)
    assert torch.all(o[:, fill_to:] == 7.0)


# The streaming sign kernel forced below its threshold (one 16-row block) and at the config-3
# shapes with their automatic split counts, against the oracle.
@pytest.mark.parametrize("m", [1, 5, 16])
def test_sign_stream_forced_small_m(dev, m, plan):
    plan("OC_SIGN_STREAM", 1)
    k, n = 1408, 720
    r, bp1, bp3, s0, s2, s4 = _factors(k, n, 1900 + m)
    x = torch.randn(m, k, generator=torch.Generator().manual_seed(m)).half()
    prep = dbf_ops.dbf_prepare(_t(s0, dev), _t(bp1, dev), _t(s2, dev), _t(bp3, dev), _t(s4, dev), k, r, n)
    y = dbf_ops.dbf_forward(x.to(dev), [prep]).float().cpu().numpy()
    ref = od.dbf_forward(x.numpy(), s0, bp1, s2, bp3, s4, k, r, n)
    assert _rel(y, ref) <= 2e-3, _rel(y, ref)


# oc_sign_gemm_batch: independent single-term problems (MDBF's per-path rank stages) in one launch —
# the sign GEMV at M <= 12, the streaming kernel at 13 <= M <= 64 (with K splits and their per-problem
# reduce at some M), one call per problem above 64 rows or when the problems' unit sizes differ.
# Every output must equal oc_sign_gemm on its problem alone, bit for bit, and the oracle.
@pytest.mark.parametrize("m", [1, 5, 13, 32, 64, 100])
@pytest.mark.parametrize("n_prob,kds,with_pre,dtype", [(2, [1000, 1000], True, "fp16"),
                                                       (3, [700, 700, 700], False, "fp16"),
                                                       (2, [1000, 1000], True, "bf16"),
                                                       (2, [1000, 300], True, "fp16")])  # last: unit sizes differ
def test_sign_gemm_batch(dev, m, n_prob, kds, with_pre, dtype):
    R, fill_to, ld_out = 530, 536, 544
    td = torch.float16 if dtype == "fp16" else torch.bfloat16
    rng = np.random.default_rng(70 + m + n_prob)
    probs, refs = [], []
    for i, kd in enumerate(kds):
        signs = rng.choice([-1, 1], size=(R, kd))
        f = dbf_ops.sign_prepare(_t(od.pack_binary(signs), dev), R, kd)
        ldx = (kd + 7) // 8 * 8
        x = torch.zeros((m, ldx), dtype=td)
        x[:, :kd] = torch.randn(m, kd, generator=torch.Generator().manual_seed(80 + i)).to(td)
        pre = None
        if with_pre:
            pre = torch.zeros(ldx, dtype=td)
            pre[:kd] = (torch.rand(kd, generator=torch.Generator().manual_seed(90 + i)) + 0.5).to(td)
        post = (torch.rand(R, generator=torch.Generator().manual_seed(100 + i)) + 0.25).to(td)
        post[torch.rand(R, generator=torch.Generator().manual_seed(110 + i)) < 0.3] *= -1
        xs = x[:, :kd].float() if pre is None else (x[:, :kd].float() * pre[:kd].float()).to(td).float()
        refs.append((xs @ torch.from_numpy(signs).float().t()) * post.float())
        probs.append((f, x.to(dev), None if pre is None else pre.to(dev), post.to(dev)))
    outs = [torch.full((m, ld_out), 7.0, dtype=td, device=dev) for _ in probs]
    dbf_ops.sign_gemm_batch(probs, m, R, td, outs, ld_out, fill_to=fill_to)
    for i, (p, o, ref) in enumerate(zip(probs, outs, refs)):
        one = torch.full((m, ld_out), 7.0, dtype=td, device=dev)
        dbf_ops.sign_gemm([p], m, R, td, one, ld_out, fill_to=fill_to)
        assert torch.equal(o, one), f"problem {i}: batched output differs from the single call"
        oc = o.float().cpu()
        assert _rel(oc[:, :R].numpy(), ref.numpy()) <= (2e-3 if dtype == "fp16" else 8e-3)
        assert torch.all(oc[:, R:fill_to] == 0) and torch.all(oc[:, fill_to:] == 7.0)
