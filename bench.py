"""Benchmark of the MI355X quantized-linear hot path (one JSON line on stdout).

Default workload: one Llama-3-8B decoder layer's seven
Mixed-GPTQ projections (q/o 4-bit, k/v 8-bit, gate/up 3-bit, down 2-bit,
group 128) at M = 1 with fp16 activations.  A step = the layer's apply()
calls over one batch as a fused-module plugin issues them: qkv_proj is one
fused module whose shards differ in bits (q 4-bit | k, v 8-bit, served with
``fused_mixed_bits`` by one grouped launch), gate|up is a merged same-bits
layer, o and down are single -- 4 launches.

- value: whole-step algorithmic bytes (packed weights + fp16 scales + packed
  zeros + x + y, each counted once) / wall time per step, with all inputs
  resident in HBM.  Weights rotate over >= 1 GiB of distinct copies so the
  256 MB Infinity Cache cannot serve them.
- roofline: the dominant kernel's algorithmic bytes / its average duration,
  measured with HIP events on the launch stream inside the timed region.
- cpu_baseline: OneComp's CPU path restated (oracle unpack + v1 restore +
  dequant to fp32, then torch.matmul on the host cores), timed on a bounded
  sample of the same step.
- secondary: M = 2048 dequant-GEMM TFLOP/s at the Qwen3-14B gate_up shape
  (config 4, bf16), the metric's second half.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0
MFMA_F16_PEAK_TFLOPS = 2500.0


def _gptq_bytes(c, m):
    return c.weight_bytes() + m * c.in_features * 2 + m * c.out_features * 2


def _prepare_copies(cases, dev, min_bytes):
    import torch

    from onecompression_amd import ops

    per = sum(c.weight_bytes() for c in cases)
    copies = max(1, -(-min_bytes // per))
    sets = []
    for i in range(copies):
        preps = []
        for c in cases:
            cd = c.to(dev)
            preps.append(ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, cd.g_idx, c.bits,
                                          c.group_size))
        sets.append(preps)
    torch.cuda.synchronize()
    return sets


def _call_name(call):
    if len(call) == 1:
        return call[0].name
    return "qkv_proj" if call[0].name == "q_proj" else "+".join(c.name for c in call)


def _replay_times(g, steps, replays):
    """Per-step ms of `replays` back-to-back replays of graph g (HIP events on the replay stream)
    and the host wall time per step of the first one (synchronised on both sides)."""
    import torch

    torch.cuda.synchronize()
    t0 = time.perf_counter()
    g.replay()
    torch.cuda.synchronize()
    wall = (time.perf_counter() - t0) / steps
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(replays)]
    for e0, e1 in evs:
        e0.record()
        g.replay()
        e1.record()
    torch.cuda.synchronize()
    return [e0.elapsed_time(e1) / steps for e0, e1 in evs], wall


def bench_gptq_layer(cfg, m, steps, warmup, dev, dtype_name="fp16", rotate_bytes=1 << 30, dispatch="fused",
                     replays=7):
    """One decoder layer's projections per step.  dispatch "fused": the apply() calls of a
    fused-module plugin (config 1: qkv_proj as one grouped launch, merged gate|up);
    "reference": every projection as its own linear, the dispatch the reference can serve
    (it rejects a qkv_proj whose shards differ in bits)."""
    import torch

    from onecompression_amd import ops, synth

    dtype = torch.float16 if dtype_name == "fp16" else torch.bfloat16
    calls = synth.layer_calls(cfg) if dispatch == "fused" else [[c] for c in synth.config_cases(cfg)]
    cases = [c for call in calls for c in call]
    flat = _prepare_copies(cases, dev, rotate_bytes)
    # per copy: the prepared parts of each call
    sets = []
    for preps in flat:
        it = iter(preps)
        sets.append([[next(it) for _ in call] for call in calls])
    xs = [synth.activations(m, call[0].in_features, dtype, seed=100 + i).to(dev) for i, call in enumerate(calls)]
    outs = [torch.empty((m, sum(c.out_features for c in call)), dtype=dtype, device=dev) for call in calls]
    step_bytes = sum(_gptq_bytes(c, m) - (2 * m * c.in_features if j else 0)
                     for call in calls for j, c in enumerate(call))  # x read once per call

    def launch(j, preps):
        if len(preps) == 1:
            ops.gptq_gemm(xs[j], preps[0], out=outs[j])
        else:
            ops.gptq_gemm_grouped(xs[j], preps, out=outs[j])

    def step(i):
        for j, preps in enumerate(sets[i % len(sets)]):
            launch(j, preps)

    for i in range(max(warmup, len(sets))):
        step(i)
    torch.cuda.synchronize()

    # The step as vLLM runs it in production: apply() calls captured in a HIP
    # graph.  The graph holds exactly `steps` steps (step i on weight copy
    # i mod copies), as a decode iteration's graph holds every layer, so no
    # graph-launch gap is charged per step.  After the eager warmup steps the
    # graph is replayed once untimed, once timed on the host clock, then
    # `replays` times with HIP events; the step time is the median replay.
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(steps):
            step(i)
    g.replay()
    per_step_ms, wall_first = _replay_times(g, steps, replays)
    wall = statistics.median(per_step_ms) * 1e-3

    # Per-call durations: for each apply() call, HIP events on the launch
    # stream around `steps` back-to-back launches of that call (rotating
    # weight copies), with the stream pre-loaded by a spin kernel so that the
    # host enqueues every launch before the GPU reaches them.
    torch.cuda._sleep(int(1e8))
    evs = []
    for j in range(len(calls)):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for i in range(steps):
            launch(j, sets[(warmup + i) % len(sets)][j])
        e1.record()
        evs.append((e0, e1))
    torch.cuda.synchronize()
    per_kernel_ms = [e0.elapsed_time(e1) / steps for e0, e1 in evs]
    kernels = []
    for call, t in zip(calls, per_kernel_ms):
        b = sum(_gptq_bytes(c, m) - (2 * m * c.in_features if j else 0) for j, c in enumerate(call))
        kernels.append({"name": _call_name(call), "bits": "|".join(str(c.bits) for c in call),
                        "K": call[0].in_features, "N": sum(c.out_features for c in call),
                        "bytes": b, "us": t * 1e3, "GBps": b / (t * 1e-3) / 1e9})
    return {"step_bytes": step_bytes, "wall_s": wall, "kernels": kernels, "copies": len(sets),
            "cases": cases, "replay_ms_per_step": per_step_ms, "wall_first_replay_s": wall_first}


def bench_gemm_large(m, steps, warmup, dev, shape=("gate_up_proj", 5120, 34816, 4)):
    import torch

    from onecompression_amd import ops, synth

    name, k, n, bits = shape
    c = synth.gptq_case(name, k, n, bits, 128, False, seed=7).to(dev)
    p = ops.gptq_prepare(c.qweight, c.qzeros, c.scales, None, bits, 128)
    x = synth.activations(m, k, torch.bfloat16, seed=8).to(dev)
    y = torch.empty((m, n), dtype=torch.bfloat16, device=dev)
    for _ in range(warmup):
        ops.gptq_gemm(x, p, out=y)
    torch.cuda.synchronize()
    # each launch between its own HIP events on the launch stream; the median launch is reported
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(steps)]
    for e0, e1 in evs:
        e0.record()
        ops.gptq_gemm(x, p, out=y)
        e1.record()
    torch.cuda.synchronize()
    times = sorted(e0.elapsed_time(e1) for e0, e1 in evs)
    ms = statistics.median(times)
    tflops = 2.0 * m * k * n / (ms * 1e-3) / 1e12
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("kernels", {}).get(f"k_gemm {name} {k}->{n} {bits}b M={m}")
    return {"workload": f"cfg4 {name} {k}->{n} {bits}b gs128 bf16", "M": m, "ms": round(ms, 4),
            "launches": steps, "ms_min_max": [round(times[0], 4), round(times[-1], 4)],
            "TFLOPs": round(tflops, 1), "frac_mfma_peak": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
            "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": MFMA_F16_PEAK_TFLOPS,
                         "unit": "TFLOP/s", "frac": round(tflops / MFMA_F16_PEAK_TFLOPS, 4),
                         "traffic": traffic, "kernel": f"k_gemm<{bits},4,true>",
                         "avg_us": round(ms * 1e3, 1)}}


RIDGE_FLOP_PER_BYTE = MFMA_F16_PEAK_TFLOPS * 1e12 / (HBM_PEAK_GBS * 1e9)

# MoE blocks with GPTQ experts (not a BASELINE config): name, hidden, intermediate, experts, top-k, Ms
MOE_SHAPES = [("Qwen3-30B-A3B experts", 2048, 768, 128, 8, (1, 8, 256, 2048)),
              ("Mixtral-8x7B experts", 4096, 14336, 8, 2, (1, 4, 64, 512))]


def report_moe(dev, bits=4, gs=128, routings=16):
    """µs per MoE block forward (oc_moe_gptq_forward: gate|up, act, down, combine) at decode M.

    Bytes: `GBps` counts each expert the routing hit once (its packed weights + fp16 scales +
    packed zeros, as a checkpoint stores them) plus x and y; `pair_GBps` counts one expert read
    per (token, slot) pair, which is what the kernels read (an expert hit by two tokens is read
    twice).  The routing cycles over `routings` seeded draws and the expert buffers over >= 1 GiB
    of copies, so the Infinity Cache cannot serve the weights."""
    import torch

    from onecompression_amd import moe, synth

    out = []
    for name, H, I, E, k, ms in MOE_SHAPES:
        g13, g2 = H // gs, I // gs
        e_bytes = (H * 2 * I * bits // 8 + g13 * 2 * I * (2 * 8 + bits) // 8
                   + I * H * bits // 8 + g2 * H * (2 * 8 + bits) // 8)
        trios = []
        for j in range(2):
            cs = [synth.gptq_case(n_, a, b, bits, gs, False, seed=900 + 3 * j + t).to(dev)
                  for t, (n_, a, b) in enumerate((("gate", H, I), ("up", H, I), ("down", I, H)))]
            trios.append([(c.qweight, c.qzeros, c.scales) for c in cs])
        copies = max(1, min(8, -(-(1 << 30) // (E * e_bytes))))
        exs = [moe.prepare_experts([trios[e % 2][0] for e in range(E)], [trios[e % 2][1] for e in range(E)],
                                   [trios[e % 2][2] for e in range(E)], bits, gs) for _ in range(copies)]
        del trios
        gen = torch.Generator().manual_seed(77)
        for m in ms:
            x = synth.activations(m, H, torch.float16, seed=600 + m).to(dev)
            rts = []
            for _ in range(routings):
                idx = torch.stack([torch.randperm(E, generator=gen)[:k] for _ in range(m)]).to(torch.int32)
                w = torch.softmax(torch.randn(m, k, generator=gen), dim=-1)
                rts.append((idx.to(dev), w.to(dev), len(set(idx.flatten().tolist()))))
            n_rot = routings * copies
            iters = 2 * n_rot if m <= 64 else 16  # prefill calls hold a large workspace each
            us = _time_graph(lambda i: moe.moe_forward(x, rts[i % routings][0], rts[i % routings][1],
                                                       exs[(i // routings) % copies]), n_rot, iters)
            distinct = sum(r[2] for r in rts) / routings
            io = 4 * m * H
            out.append({"block": name, "H": H, "I": I, "E": E, "topk": k, "bits": bits, "gs": gs, "M": m,
                        "dtype": "fp16", "us": round(us, 2), "experts_hit": round(distinct, 2),
                        "GBps": round((distinct * e_bytes + io) / (us * 1e-6) / 1e9, 1),
                        "pair_GBps": round((m * k * e_bytes + io) / (us * 1e-6) / 1e9, 1),
                        "TFLOPs": round(2.0 * m * k * 3 * H * I / (us * 1e-6) / 1e12, 2),
                        "frac_hbm_peak": round((distinct * e_bytes + io) / (us * 1e-6) / 1e9 / HBM_PEAK_GBS, 4)})
        del exs
        torch.cuda.empty_cache()
    return out


def _time_graph(launch, copies, iters, warm=2):
    """µs per launch: `iters` launches (launch(i) uses copy i % copies) in one HIP graph, the median of
    three timed replays.  Every copy runs once before the capture (as every layer of a served model
    has run once): a layer's first call builds its cached operands (the DBF/MDBF scale vectors in the
    activation dtype), which must not be captured into the graph and re-run on each replay."""
    import torch

    for i in range(max(warm, copies)):
        launch(i)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        for i in range(iters):
            launch(i)
    g.replay()
    torch.cuda.synchronize()
    evs = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(3)]
    for e0, e1 in evs:
        e0.record()
        g.replay()
        e1.record()
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in evs) * 1e3 / iters


def _entry(cfg, name, k, n, m, bits, nbytes, flops, us, dtype):
    gbs = nbytes / (us * 1e-6) / 1e9
    tfs = flops / (us * 1e-6) / 1e12
    bound = "hbm" if flops / nbytes < RIDGE_FLOP_PER_BYTE else "mfma"
    return {"cfg": cfg, "layer": name, "K": k, "N": n, "bits": bits, "M": m, "dtype": dtype,
            "us": round(us, 2), "GBps": round(gbs, 1), "frac_hbm_peak": round(gbs / HBM_PEAK_GBS, 4),
            "TFLOPs": round(tfs, 2), "frac_mfma_peak": round(tfs / MFMA_F16_PEAK_TFLOPS, 4), "bound": bound}


def _rotation(weight_bytes, ms, rotate_bytes=1 << 30):
    """Weight copies for a layer: enough to exceed the MALL when any M is HBM-bound."""
    return max(1, min(32, -(-rotate_bytes // weight_bytes))) if min(ms) <= 64 else 1


def report_configs(dev, only=None):
    """BASELINE configs 0-4 at every listed M: µs per apply(), GB/s, TFLOP/s, binding roof."""
    import torch

    from onecompression_amd import dbf_ops, ops, synth

    out = []
    plan = [(0, synth.config_cases(0), (1, 16), torch.float16),
            (1, synth.layer_cases(1), (1, 8, 32, 128), torch.float16),
            (2, synth.config_cases(2), (1, 16, 64, 256), torch.float16),
            (4, synth.config_cases(4), (2048, 4096, 8192), torch.bfloat16)]
    plan = [p for p in plan if only is None or p[0] in only]
    for cfg, cases, ms, dt in plan:
        dname = "fp16" if dt == torch.float16 else "bf16"
        for c in cases:
            cd = c.to(dev)
            p0 = ops.gptq_prepare(cd.qweight, cd.qzeros, cd.scales, cd.g_idx, c.bits, c.group_size)
            del cd
            preps = [p0] + [ops.PreparedGPTQ(p0.packed.clone(), p0.meta.clone(), p0.perm, p0.in_features,
                                             p0.out_features, p0.bits, p0.group_size, p0.num_groups)
                            for _ in range(_rotation(c.weight_bytes(), ms) - 1)]
            for m in ms:
                x = synth.activations(m, c.in_features, dt, seed=200 + m).to(dev)
                y = torch.empty((m, c.out_features), dtype=dt, device=dev)
                iters = 64 if m <= 256 else 8
                us = _time_graph(lambda i: ops.gptq_gemm(x, preps[i % len(preps)], out=y), len(preps), iters)
                out.append(_entry(cfg, c.name, c.in_features, c.out_features, m, c.bits,
                                  _gptq_bytes(c, m), 2.0 * m * c.in_features * c.out_features, us, dname))
            del preps, p0
            torch.cuda.empty_cache()
    # online Hadamard of a rotated down_proj input (configs 1, 2, 4 intermediate sizes)
    if only is None or only & {1, 2, 4}:
        for cfg, n_dim, dt, ms in ((1, 14336, torch.float16, (1, 128)), (2, 12288, torch.float16, (1, 256)),
                                   (4, 17408, torch.bfloat16, (2048,))):
            if only is not None and cfg not in only:
                continue
            for m in ms:
                x = synth.activations(m, n_dim, dt, seed=500 + m).to(dev)
                y = torch.empty_like(x)
                # the reference's default rounding (fp32_had=False, pure-PyTorch transform: every
                # butterfly stage rounded) and the fused-transform-op rounding (one rounding)
                for rnd in ("stages", "once"):
                    us = _time_graph(lambda i: ops.hadamard(x, out=y, rounding=rnd), 1, 64 if m <= 256 else 16)
                    k_blk = ops.hadamard_order(n_dim)
                    fl = 2.0 * m * n_dim * (k_blk + math.log2(n_dim // k_blk))
                    out.append(_entry(cfg, f"hadamard n={n_dim} (K={k_blk}) rounding={rnd}", n_dim, n_dim, m, 0,
                                      4 * m * n_dim, fl, us, "fp16" if dt == torch.float16 else "bf16"))
    # config 3: one DBF path and the two-path MDBF variant, per shape
    for i, (name, k, n) in enumerate(synth.CONFIG3 if only is None or 3 in only else []):
        cases = [synth.dbf_case(name, k, n, 1.0, seed=300 + 2 * i + j) for j in range(2)]
        ms = (1, 32, 512)
        copies = _rotation(sum(c.weight_bytes() for c in cases), ms)
        parts, paths = [], []
        for rep in range(copies):
            row_p, row_m = [], []
            for c in cases:
                cd = c.to(dev)
                row_p.append(dbf_ops.dbf_prepare(cd.s0, cd.bp1, cd.s2, cd.bp3, cd.s4, k, c.mid, n))
                row_m.append(dbf_ops.mdbf_prepare_path(
                    cd.bp3, (n, c.mid), cd.bp1, (c.mid, k), cd.s4.view(n, 1), cd.s0.view(k, 1),
                    cd.s2.view(c.mid, 1), torch.ones((c.mid, 1), dtype=torch.float16, device=dev)))
            parts.append(row_p[0])
            paths.append(row_m)
        for m in ms:
            x = synth.activations(m, k, torch.float16, seed=400 + m).to(dev)
            iters = 64 if m <= 32 else 16
            c = cases[0]
            byt = c.weight_bytes() + 2 * m * (k + n)
            fl = 2.0 * m * c.mid * (k + n)
            us = _time_graph(lambda j: dbf_ops.dbf_forward(x, [parts[j % copies]]), copies, iters)
            out.append(_entry(3, f"dbf {name}", k, n, m, 1, byt, fl, us, "fp16"))
            byt2 = sum(cc.weight_bytes() for cc in cases) + 2 * m * (k + n)
            us = _time_graph(lambda j: dbf_ops.mdbf_forward(x, paths[j % copies]), copies, iters)
            out.append(_entry(3, f"mdbf P=2 {name}", k, n, m, 1, byt2, 2 * fl, us, "fp16"))
        del parts, paths
        torch.cuda.empty_cache()
    return out


def _cpu_model():
    """The host CPU as lscpu names it (model name, family/model/stepping, sockets x cores x threads)."""
    import subprocess

    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
    except (OSError, subprocess.SubprocessError):
        out = ""
    f = {}
    for line in out.splitlines():
        if ":" in line:
            k, v = line.split(":", 1)
            f[k.strip()] = v.strip()
    if "Model name" not in f:
        try:
            with open("/proc/cpuinfo") as fh:
                for line in fh:
                    if line.startswith("model name"):
                        return line.split(":", 1)[1].strip()
        except OSError:
            pass
        return "unknown"
    return (f"{f['Model name']} (family {f.get('CPU family', '?')} model {f.get('Model', '?')} stepping "
            f"{f.get('Stepping', '?')}; {f.get('Socket(s)', '?')} socket(s) x {f.get('Core(s) per socket', '?')} "
            f"cores x {f.get('Thread(s) per core', '?')} threads)")


def cpu_baseline(cases, m, budget_s=20.0, min_runs=3, max_runs=10, warmup=1):
    """OneComp's CPU path (checkpoint.py:186-259 + torch.matmul) on the host cores.

    Per run: for every layer, the oracle's unpack + v1 zero restore + fp32
    dequant (timed as `dequant`), then torch.matmul(x, W.T) in fp32 (`matmul`).
    Runs stop at max_runs or once budget_s is spent (never below min_runs).
    """
    import numpy as np
    import torch

    from oracle import gptq as og

    torch.set_num_threads(os.cpu_count() or 1)
    threads = torch.get_num_threads()
    x = [torch.from_numpy(np.random.default_rng(i).normal(size=(m, c.in_features)).astype(np.float32))
         for i, c in enumerate(cases)]

    def run():
        td = tm = 0.0
        for c, xi in zip(cases, x):
            t0 = time.perf_counter()
            qw, qz, sc = c.qweight.numpy(), c.qzeros.numpy(), c.scales.numpy()
            q = og.unpack_int_weights(qw, c.bits, (c.out_features, c.in_features))
            z = og.restore_zeros(og.unpack_zeros(qz, c.bits, c.out_features), c.bits, "gptq")
            g = og.default_g_idx(c.in_features, c.group_size) if c.g_idx is None else c.g_idx.numpy()
            w = torch.from_numpy(og.dequant_fp32(q, sc, z, g))
            t1 = time.perf_counter()
            torch.matmul(xi, w.T)
            td += t1 - t0
            tm += time.perf_counter() - t1
        return td, tm

    for _ in range(warmup):
        run()
    runs = []
    t_start = time.perf_counter()
    while len(runs) < max_runs and (len(runs) < min_runs or time.perf_counter() - t_start < budget_s):
        runs.append(run())
    tot = statistics.median(d + mm for d, mm in runs)
    step_bytes = sum(_gptq_bytes(c, m) for c in cases)
    return {"value": step_bytes / tot / 1e9, "unit": "GB/s", "cores": threads, "kind": "port",
            "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "median_s": round(tot, 4), "dequant_s": round(statistics.median(d for d, _ in runs), 4),
            "matmul_s": round(statistics.median(mm for _, mm in runs), 4), "runs": len(runs),
            "warmup": warmup,
            "sample": f"{len(runs)} full step(s) after {warmup} warmup of the same workload "
                      f"({len(cases)} layers, M={m}); numpy unpack + v1 restore + fp32 dequant, then "
                      f"torch.matmul fp32 on {threads} threads"}


def cpu_baseline_dbf(m, runs=10, warmup=2):
    """DoubleBinaryLinear.forward restated on the host (dbf_layer.py:251-268): unpack the two sign
    factors (oracle), then x*s0 -> @S2^T -> *s2 -> @S1^T -> *s4 as fp32 torch matmuls; config 3
    up_proj shape, one path."""
    import numpy as np
    import torch

    from oracle import dbf as od
    from onecompression_amd import synth

    torch.set_num_threads(os.cpu_count() or 1)
    name, k, n = synth.CONFIG3[0]
    c = synth.dbf_case(name, k, n, 1.0, seed=300)
    x = torch.from_numpy(np.random.default_rng(1).normal(size=(m, k)).astype(np.float32))
    s0, s2, s4 = (v.float() for v in (c.s0, c.s2, c.s4))

    def run():
        t0 = time.perf_counter()
        S2 = torch.from_numpy(od.unpack_binary_factor(c.bp1.numpy(), (c.mid, k)).astype(np.float32))
        S1 = torch.from_numpy(od.unpack_binary_factor(c.bp3.numpy(), (n, c.mid)).astype(np.float32))
        t1 = time.perf_counter()
        (((x * s0) @ S2.T) * s2 @ S1.T) * s4
        return t1 - t0, time.perf_counter() - t1

    for _ in range(warmup):
        run()
    rs = [run() for _ in range(runs)]
    tot = statistics.median(a + b for a, b in rs)
    nbytes = c.weight_bytes() + 2 * m * (k + n)
    return {"value": nbytes / tot / 1e9, "unit": "GB/s", "cores": torch.get_num_threads(), "kind": "port",
            "cpu_model": _cpu_model(), "median_s": round(tot, 4),
            "unpack_s": round(statistics.median(a for a, _ in rs), 4),
            "matmul_s": round(statistics.median(b for _, b in rs), 4), "runs": runs, "warmup": warmup,
            "sample": f"config 3 {name} {k}->{n} (r={c.mid}), one DBF path, M={m}: oracle unpack of both "
                      f"sign factors + fp32 torch matmuls, {torch.get_num_threads()} threads"}


def synth_config0():
    from onecompression_amd import synth

    return synth.config_cases(0)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--config", type=int, default=1)
    ap.add_argument("--m", type=int, default=1)
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--no-secondary", action="store_true")
    ap.add_argument("--no-configs", action="store_true",
                    help="skip the per-config report (BASELINE configs 0-4 at every M)")
    ap.add_argument("--configs-only", type=str, default=None,
                    help="comma-separated BASELINE configs: print only their per-config report")
    ap.add_argument("--gemm-only", action="store_true",
                    help="only the M=2048 dequant-GEMM measurement (config 4 gate_up, bf16)")
    ap.add_argument("--moe-only", action="store_true",
                    help="only the MoE block report (GPTQ experts at decode M)")
    ap.add_argument("--no-moe", action="store_true", help="skip the MoE block report")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="only run a 256 MiB device copy (reference kernel for HBM byte counters)")
    args = ap.parse_args()
    if args.gpus != 1:
        print("bench.py measures one GPU only (the multi-GPU path is not part of this build); "
              "run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.calibrate_copy:
        n = 256 << 20
        src = torch.ones(n, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(5):
            dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"calibration": "device copy", "bytes_read": n, "bytes_written": n, "launches": 5}))
        return
    if args.configs_only is not None:
        print(json.dumps({"configs": report_configs(dev, {int(c) for c in args.configs_only.split(",")})}))
        return
    if args.gemm_only:
        print(json.dumps(bench_gemm_large(2048, args.steps, args.warmup, dev)))
        return
    if args.moe_only:
        print(json.dumps({"moe": report_moe(dev)}))
        return
    r = bench_gptq_layer(args.config, args.m, args.steps, args.warmup, dev)
    ref_dispatch = None
    if args.config == 1:
        # the same layer with every projection as its own linear (what the reference can serve: it
        # rejects a qkv_proj whose shards differ in bits); weights of the fused run freed first
        torch.cuda.empty_cache()
        rr = bench_gptq_layer(args.config, args.m, args.steps, args.warmup, dev, dispatch="reference")
        ref_dispatch = {"value": round(rr["step_bytes"] / rr["wall_s"] / 1e9, 1), "unit": "GB/s",
                        "ms_per_step": round(rr["wall_s"] * 1e3, 4),
                        "frac_hbm_peak": round(rr["step_bytes"] / rr["wall_s"] / 1e9 / HBM_PEAK_GBS, 4),
                        "calls": "q_proj, k_proj, v_proj, o_proj, gate_proj, up_proj, down_proj (7 launches)",
                        "replay_ms_per_step": [round(v, 5) for v in rr["replay_ms_per_step"]],
                        "per_kernel": [{k: (round(v, 2) if isinstance(v, float) else v) for k, v in kk.items()}
                                       for kk in rr["kernels"]]}
        del rr
        torch.cuda.empty_cache()
    dom = max(r["kernels"], key=lambda k: k["us"])
    value = r["step_bytes"] / r["wall_s"] / 1e9
    # the wide dominant layer's kernel at M <= 4 (k_gemv_stream_bal at M >= 3 when its n-tiles load
    # the CUs unevenly, as config 1's gate|up does); other M name the call only
    cus = torch.cuda.get_device_properties(dev).multi_processor_count
    kern = "dominant call"
    if args.m <= 4:
        kern = "k_gemv_stream" if args.m <= 2 or (dom["N"] // 16) % (4 * cus) == 0 else "k_gemv_stream_bal"
    kname = f"{kern} {dom['name']} {dom['K']}->{dom['N']} {dom['bits']}b"
    traffic = None
    tpath = os.path.join(ROOT, "profiles", "traffic.json")
    if os.path.exists(tpath):
        with open(tpath) as f:
            traffic = json.load(f).get("kernels", {}).get(kname)
    out = {
        "metric": "M=1 dequant-GEMV HBM GB/s (%peak); M=2048 dequant-GEMM TFLOP/s (%MFMA peak)",
        "value": round(value, 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(r["wall_s"] * 1e3, 4),
        "timing": {"method": f"median of {len(r['replay_ms_per_step'])} replays (HIP events) of a graph "
                             f"of {args.steps} steps",
                   "replay_ms_per_step": [round(v, 5) for v in r["replay_ms_per_step"]],
                   "first_replay_host_clock_ms_per_step": round(r["wall_first_replay_s"] * 1e3, 5)},
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic (seeded uniform codes/zeros, |N(0,0.02)|+1e-3 scales, N(0,1) x)",
        "config": {"workload": f"cfg{args.config} Llama-3-8B decoder layer, 7 Mixed-GPTQ projections "
                               f"(q,o 4b; k,v 8b; gate,up 3b; down 2b; gs128) as 4 apply() calls: "
                               f"qkv_proj (q 4b | k,v 8b in one grouped launch), o_proj, gate_up_proj, "
                               f"down_proj, M={args.m}, fp16",
                   "M": args.m, "frac_hbm_peak": round(value / HBM_PEAK_GBS, 4),
                   "weight_copies_rotated": r["copies"]},
        "roofline": {"bound": "hbm", "achieved": round(dom["GBps"], 1), "peak": HBM_PEAK_GBS,
                     "unit": "GB/s", "frac": round(dom["GBps"] / HBM_PEAK_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": dom["bytes"], "kernel": kname, "avg_us": round(dom["us"], 2),
                     "traffic_source": "profiles/traffic.json (rocprofv3 --pmc, copy-calibrated)"},
        "per_kernel": [{k: (round(v, 2) if isinstance(v, float) else v) for k, v in kk.items()}
                       for kk in r["kernels"]],
    }
    if ref_dispatch is not None:
        out["reference_dispatch"] = ref_dispatch
    if not args.no_secondary:
        try:
            out["secondary"] = bench_gemm_large(2048, 21, 3, dev)
        except Exception as e:  # the large-M measurement is reported, never hides the main line
            out["secondary"] = {"error": str(e)}
    if not args.no_configs:
        try:
            out["configs"] = report_configs(dev)
        except Exception as e:  # reported, never hides the main line
            out["configs"] = {"error": str(e)}
    if not args.no_moe:
        try:
            out["moe"] = report_moe(dev)
        except Exception as e:  # reported, never hides the main line
            out["moe"] = {"error": str(e)}
    if not args.no_cpu:
        out["cpu_baseline"] = cpu_baseline(r["cases"], args.m, budget_s=0.0, min_runs=10, max_runs=10, warmup=2)
        c0 = synth_config0()
        out["cpu_baseline_cfg0"] = {f"M={mm}": cpu_baseline(c0, mm, budget_s=15.0, min_runs=10, max_runs=10,
                                                             warmup=2) for mm in (1, 16)}
        out["cpu_baseline_cfg3"] = {f"M={mm}": cpu_baseline_dbf(mm) for mm in (1, 32)}
    print(json.dumps(out))


if __name__ == "__main__":
    main()
