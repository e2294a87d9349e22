"""Host model of the MoE prefill plan (CPU).

Models the tables `k_moe_sort` builds and the tile grid `moe_prefill` launches over them
(onecompression_amd/csrc/gptq_gemm.hip). It checks the invariants the grouped `k_gemm` relies
on: every run gets a workgroup row of the grid, the runs partition the valid pairs expert by
expert, and no run is taller than the tile. Cases:
- the shape of the one unexplained prefill mismatch (E = 4, H = 256, I = 160, top-2, M = 130,
  ids with -1 and E, the routing of tests/test_gpu_moe.py::test_moe_prefill_gemm);
- routings built to maximise the number of runs.
The model restates the host formulas; it pins them against these invariants, not against the
kernel's output (the GPU tests do that).
"""

import numpy as np
import pytest
import torch


def plan_model(ids, E, gs13=128, gs2=128):
    """(BM, tiles, runs, cnt, off) for ids [M, topk]: moe_prefill's tile height 64 MT (MT from
    the pairs per busy expert; 256-row tiles for groups below 128) and grid bound, and
    k_moe_sort's per-expert counts, offsets and runs {expert, first sorted row, rows}."""
    M, topk = ids.shape
    pairs = M * topk
    busy = min(E, pairs)
    avg = pairs // busy
    mt = 4 if avg >= 256 else (2 if avg >= 128 else 1)
    if gs13 % 128 or gs2 % 128:
        mt = 4
    BM = 64 * mt
    tiles = min((pairs + BM - 1) // BM + busy, pairs)
    flat = ids.reshape(-1)
    valid = (flat >= 0) & (flat < E)
    cnt = np.bincount(flat[valid], minlength=E)
    off = np.concatenate([[0], np.cumsum(cnt)[:-1]])
    runs = [(e, int(off[e]) + BM * i, int(min(BM, cnt[e] - BM * i)))
            for e in range(E) for i in range((int(cnt[e]) + BM - 1) // BM)]
    return BM, tiles, runs, cnt, off


def check_plan(ids, E, gs13=128, gs2=128):
    BM, tiles, runs, cnt, off = plan_model(ids, E, gs13, gs2)
    assert len(runs) <= tiles, (len(runs), tiles)  # every run has its row of workgroups
    nxt = 0
    for e, first, rows in runs:  # expert order, contiguous, inside the expert's range
        assert first == nxt and 1 <= rows <= BM, (e, first, rows)
        assert off[e] <= first and first + rows <= off[e] + cnt[e]
        nxt = first + rows
    assert nxt == int(cnt.sum())  # every valid pair in exactly one run
    return BM, tiles, runs


def test_plan_of_the_unexplained_case():
    E, H, I, k, m = 4, 256, 160, 2, 130
    g = torch.Generator().manual_seed(22)  # the GPU test's routing
    idx = torch.stack([torch.randperm(E, generator=g)[:k] for _ in range(m)]).to(torch.int32).numpy()
    idx[3, 0] = -1
    idx[4, :] = E
    BM, tiles, runs = check_plan(idx, E)
    assert BM == 64  # 64-row tiles (65 pairs per busy expert)
    assert sum(r[2] for r in runs) == m * k - 3  # three invalid slots left out
    # the down GEMM's K = I = 160: its last k-block (128..255) masks 16-byte chunks from k = 160
    # on; 160 is a multiple of 8, so no chunk straddles K and the masked chunks read zero whole
    assert I % 8 == 0 and H % 128 == 0


@pytest.mark.parametrize("E,topk,m", [(4, 2, 130), (8, 2, 513), (128, 8, 2048), (16, 4, 256), (2048, 1, 4096)])
def test_plan_random_routings(E, topk, m):
    rng = np.random.default_rng(E * 1000 + m)
    for _ in range(20):
        ids = np.stack([rng.permutation(E)[:topk] for _ in range(m)]).astype(np.int64)
        bad = rng.random(ids.shape) < 0.05
        ids[bad] = rng.choice([-1, E], size=int(bad.sum()))
        check_plan(ids, E)


@pytest.mark.parametrize("gs", [128, 64])
def test_plan_worst_case_runs(gs):
    """Every expert one row past a tile boundary (two runs each), and one expert holding all
    pairs: the grid bound still covers every run."""
    E = 8
    BM = plan_model(np.zeros((64, 2), np.int64), E, gs, gs)[0]
    per = BM + 1
    ids = np.repeat(np.arange(E), per)
    ids = ids[np.random.default_rng(0).permutation(ids.size)].reshape(-1, 1)
    check_plan(ids, E, gs, gs)
    check_plan(np.zeros((300, 2), np.int64), E, gs, gs)
    check_plan(np.full((50, 2), -1, np.int64), E, gs, gs)
