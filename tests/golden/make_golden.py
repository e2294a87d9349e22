"""Writes the small golden fixtures of tests/golden/ from the oracle.

Each fixture holds seeded checkpoint-layout inputs and the oracle's outputs:
unpacked codes, restored zeros, the dequantised fp16 and bf16 weights (bit
patterns) and the fp32 GEMM output; for DBF the unpacked signs and the fp32
forward.  Regenerate with ``python tests/golden/make_golden.py``.
"""

import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.dirname(os.path.dirname(HERE)))

from oracle import dbf as od  # noqa: E402
from oracle import gptq as og  # noqa: E402


def gptq_fixture(bits, act_order, seed):
    rng = np.random.default_rng(seed)
    k, n, gs, m = 256, 64, 64, 3
    g = k // gs
    qweight = rng.integers(-(2**31), 2**31, (k * bits // 32, n), dtype=np.int64).astype(np.int32)
    qzeros = rng.integers(-(2**31), 2**31, (g, n * bits // 32), dtype=np.int64).astype(np.int32)
    scales = (np.abs(rng.normal(0, 0.02, (g, n))) + 1e-3).astype(np.float16)
    g_idx = og.g_idx_from_perm(rng.permutation(k), gs) if act_order else og.default_g_idx(k, gs)
    x = rng.normal(size=(m, k)).astype(np.float16)
    codes = og.unpack_int_weights(qweight, bits, (n, k))
    zeros = og.restore_zeros(og.unpack_zeros(qzeros, bits, n), bits, "gptq")
    w16 = og.dequantize(qweight, qzeros, scales, g_idx, bits, "gptq", "fp16")
    wbf = og.dequantize(qweight, qzeros, scales, g_idx, bits, "gptq", "bf16")
    y = og.linear_ref(x, w16, "fp16")
    return dict(bits=bits, group_size=gs, qweight=qweight, qzeros=qzeros, scales=scales, g_idx=g_idx,
                x=x, codes=codes.astype(np.uint8), zeros=zeros.astype(np.uint8), w16=w16.view(np.uint16),
                wbf16=wbf, y=y)


def dbf_fixture(seed):
    rng = np.random.default_rng(seed)
    k, n, m = 96, 40, 2
    r = od.mid_features(1.0, k, n)
    s2m, s1m = rng.choice([-1, 1], size=(r, k)), rng.choice([-1, 1], size=(n, r))
    bp1, bp3 = od.pack_binary(s2m), od.pack_binary(s1m)
    s0, s2, s4 = [(np.abs(rng.normal(0, 0.05, d)) + 1e-3).astype(np.float16) for d in (k, r, n)]
    x = rng.normal(size=(m, k)).astype(np.float16)
    y = od.dbf_forward(x, s0, bp1, s2, bp3, s4, k, r, n)
    return dict(k=k, n=n, r=r, bp1=bp1, bp3=bp3, s0=s0, s2=s2, s4=s4, x=x, S2=s2m.astype(np.int8),
                S1=s1m.astype(np.int8), y=y)


def main():
    for bits in (2, 3, 4, 8):
        for act in (False, True):
            np.savez(os.path.join(HERE, f"gptq_b{bits}_{'act' if act else 'seq'}.npz"),
                     **gptq_fixture(bits, act, 1000 + 10 * bits + act))
    np.savez(os.path.join(HERE, "dbf_k96_n40.npz"), **dbf_fixture(7))


if __name__ == "__main__":
    main()
