"""HIP graph capture of every forward entry point: each case is captured once and replayed three
times, with new inputs copied in eagerly between replays; every replay must equal the eager
result bit for bit (the kernels are deterministic, including the MoE sort's grouping)."""

import pytest
import torch

from onecompression_amd import dbf_ops, moe, ops, synth

pytestmark = pytest.mark.gpu


def _replays(dev, make_inputs, run, n=3):
    """make_inputs(i) -> list of tensors (CPU); run(list of device tensors) -> output tensor."""
    bufs = [t.to(dev) for t in make_inputs(0)]
    run(bufs)  # warm-up on the side stream torch uses for capture
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        out = run(bufs)
    for i in range(1, n + 1):
        new = make_inputs(i)
        for b, t in zip(bufs, new):
            b.copy_(t)
        want = run([t.to(dev) for t in new]).clone()  # eager, on fresh tensors
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, want), f"replay {i} differs from eager"


@pytest.mark.parametrize("k,n,bits,m,dt", [
    (4096, 28672, 3, 1, torch.float16),   # streaming GEMV (wide)
    (4096, 28672, 3, 4, torch.float16),   # balanced streaming GEMV (wide, uneven CU load)
    (4096, 4096, 4, 1, torch.float16),    # k_gemv
    (1024, 16384, 2, 24, torch.float16),  # streaming GEMM (mid M)
    (4096, 4096, 4, 128, torch.float16),  # streaming GEMM, 8 row blocks, K split + reduce
    (14336, 4096, 2, 48, torch.bfloat16), # streaming GEMM, 4 row blocks, long K split
    (512, 1024, 8, 40, torch.bfloat16),   # skinny / split-K
    (1024, 1024, 4, 300, torch.bfloat16), # large-M GEMM
])
def test_gptq_gemm_graph(dev, k, n, bits, m, dt):
    c = synth.gptq_case("g", k, n, bits, 128, False, seed=bits + m).to(dev)
    prep = ops.gptq_prepare(c.qweight, c.qzeros, c.scales, None, bits, 128)
    _replays(dev, lambda i: [synth.activations(m, k, dt, seed=40 + i)], lambda b: ops.gptq_gemm(b[0], prep))


def test_gptq_grouped_graph(dev):
    parts = [synth.gptq_case(nm, 4096, nn, bb, 128, False, seed=s).to(dev)
             for nm, nn, bb, s in (("q", 4096, 4, 1), ("k", 1024, 8, 2), ("v", 1024, 8, 3))]
    preps = [ops.gptq_prepare(c.qweight, c.qzeros, c.scales, None, c.bits, 128) for c in parts]
    _replays(dev, lambda i: [synth.activations(1, 4096, torch.float16, seed=50 + i)],
             lambda b: ops.gptq_gemm_grouped(b[0], preps))


@pytest.mark.parametrize("m", [1, 64, 200])
def test_dbf_and_mdbf_graph(dev, m):
    c = synth.dbf_case("d", 1024, 2048, 1.0, seed=5).to(dev)
    part = dbf_ops.dbf_prepare(c.s0, c.bp1, c.s2, c.bp3, c.s4, c.in_features, c.mid, c.out_features)
    _replays(dev, lambda i: [synth.activations(m, 1024, torch.float16, seed=60 + i)],
             lambda b: dbf_ops.dbf_forward(b[0], [part]))
    n_, k_ = c.out_features, c.in_features
    path = dbf_ops.mdbf_prepare_path(c.bp3, (n_, c.mid), c.bp1, (c.mid, k_), c.s4.view(n_, 1),
                                     c.s0.view(k_, 1), c.s2.view(c.mid, 1),
                                     torch.ones((c.mid, 1), dtype=torch.float16, device=dev))
    _replays(dev, lambda i: [synth.activations(m, 1024, torch.float16, seed=70 + i)],
             lambda b: dbf_ops.mdbf_forward(b[0], [path]))
    # two paths: one sign GEMM over both terms' k-blocks above 16 rows
    _replays(dev, lambda i: [synth.activations(m, 1024, torch.float16, seed=75 + i)],
             lambda b: dbf_ops.mdbf_forward(b[0], [path, path]))


@pytest.mark.parametrize("rounding", ["stages", "once", "fp32"])
def test_hadamard_graph(dev, rounding):
    _replays(dev, lambda i: [synth.activations(3, 14336, torch.float16, seed=80 + i)],
             lambda b: ops.hadamard(b[0], rounding=rounding))


@pytest.mark.parametrize("m", [1, 6, 100])
def test_moe_graph(dev, m):
    E, H, I, k = 6, 256, 128, 2
    trios = []
    for e in range(E):
        cs = [synth.gptq_case(nm, a, b, 4, 128, False, seed=90 + 3 * e + j).to(dev)
              for j, (nm, a, b) in enumerate((("g", H, I), ("u", H, I), ("d", I, H)))]
        for cc in cs:
            cc.scales = cc.scales * 0.25
        trios.append([(cc.qweight, cc.qzeros, cc.scales) for cc in cs])
    ex = moe.prepare_experts([t[0] for t in trios], [t[1] for t in trios], [t[2] for t in trios], 4, 128)

    def inputs(i):
        gen = torch.Generator().manual_seed(100 + i)
        idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(m)]).to(torch.int32)
        return [synth.activations(m, H, torch.float16, seed=110 + i), idx,
                torch.softmax(torch.randn(m, k, generator=gen), dim=-1)]

    _replays(dev, inputs, lambda b: moe.moe_forward(b[0], b[1], b[2], ex, "silu"))


def test_dbf_first_call_captured(dev):
    """A freshly prepared DBF layer and MDBF path whose first call is made under capture: every
    operand the forward reads was built at prepare time (none in the graph's private pool), so the
    replays and later eager calls (after the graph is freed) equal a fresh eager call."""
    c = synth.dbf_case("d", 1024, 2048, 1.0, seed=8).to(dev)
    part = dbf_ops.dbf_prepare(c.s0, c.bp1, c.s2, c.bp3, c.s4, c.in_features, c.mid, c.out_features)
    n_, k_ = c.out_features, c.in_features
    path = dbf_ops.mdbf_prepare_path(c.bp3, (n_, c.mid), c.bp1, (c.mid, k_), c.s4.view(n_, 1),
                                     c.s0.view(k_, 1), c.s2.view(c.mid, 1),
                                     torch.ones((c.mid, 1), dtype=torch.float16, device=dev))
    for m in (1, 32):
        x = synth.activations(m, 1024, torch.float16, seed=90 + m).to(dev)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            y = dbf_ops.dbf_forward(x, [part])
            y2 = dbf_ops.mdbf_forward(x, [path, path])
        g.replay()
        torch.cuda.synchronize()
        got, got2 = y.clone(), y2.clone()
        del g, y, y2
        torch.cuda.empty_cache()
        assert torch.equal(got, dbf_ops.dbf_forward(x, [part]))
        assert torch.equal(got2, dbf_ops.mdbf_forward(x, [path, path]))
