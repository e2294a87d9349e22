"""Pins for the GPTQ oracle (CPU only).

Each check is independent of the oracle's own formula: the reference's
known-answer tests restated, a big-integer bit-stream brute force, exact
rational arithmetic for the rounding, and torch's own bf16 cast.  A few tests
plant a plausible mistake in a copy of the oracle and show a pin catches it.
"""

from fractions import Fraction

import numpy as np
import pytest

from oracle import gptq as og

BITS = [2, 3, 4, 8]


def _rng(seed=0):
    return np.random.default_rng(seed)


@pytest.mark.parametrize("bits", BITS)
def test_minus_one_at_every_slot_round_trips(bits):
    """Restates test_gptq_layer_pack.py:122-150: -1 at any slot (incl. the
    3-bit straddle slots 10 and 21) reads back as 2^b-1, neighbours intact."""
    pf = 32 if bits == 3 else 32 // bits
    cols, mask = 3, (1 << bits) - 1
    other = min(mask - 1, 5)
    for pos in range(pf):
        values = np.full((pf, cols), other, dtype=np.int32)
        values[pos, :] = -1
        packed = og.pack_zeros(values.T, bits)  # packs along the pf axis
        unpacked = og.unpack_zeros(packed, bits, pf).T
        expected = values.copy()
        expected[pos, :] = mask
        assert np.array_equal(unpacked, expected), (bits, pos)


def _bitstream_codes(qweight_col_words, bits, k):
    """Independent restatement: one column's words form a little-endian bit
    stream (3 words per 32 codes for 3-bit, one word per 32/b codes
    otherwise); code i is (stream >> (b*i)) & mask, using Python big ints."""
    words = [int(w) & 0xFFFFFFFF for w in qweight_col_words]
    stream = 0
    for i, w in enumerate(words):
        stream |= w << (32 * i)
    return [(stream >> (bits * i)) & ((1 << bits) - 1) for i in range(k)]


@pytest.mark.parametrize("bits", BITS)
def test_unpack_matches_bitstream_brute_force(bits):
    rng = _rng(bits)
    k, n = 96 if bits == 3 else 64, 5
    qweight = rng.integers(-(2**31), 2**31, size=(k * bits // 32, n), dtype=np.int64).astype(np.int32)
    codes = og.unpack_int_weights(qweight, bits, (n, k))
    for col in range(n):
        assert codes[col].tolist() == _bitstream_codes(qweight[:, col], bits, k)


@pytest.mark.parametrize("bits", BITS)
def test_pack_unpack_round_trip(bits):
    rng = _rng(10 + bits)
    n, k, g = 48 if bits != 3 else 64, 256, 4
    q = rng.integers(0, 1 << bits, size=(n, k)).astype(np.int32)
    z = rng.integers(0, 1 << bits, size=(g, n)).astype(np.int32)
    qw = og.pack_int_weights(q, bits)
    assert qw.shape == (k * bits // 32, n) and qw.dtype == np.int32
    assert np.array_equal(og.unpack_int_weights(qw, bits, (n, k)), q)
    qz = og.pack_zeros(z, bits)
    assert qz.shape == (g, n * bits // 32)
    assert np.array_equal(og.unpack_zeros(qz, bits, n), z)


def _probe_layer(bits, fmt):
    """test_gptq_layer_pack.py:338-392: qweight=0, scale=1, one-hot x; the
    first 4 columns have raw zero 0 (stored v1 as -1), the rest raw zero 1."""
    k = n = 32
    q = np.zeros((n, k), dtype=np.int32)
    raw = np.ones((1, n), dtype=np.int32)
    raw[:, :4] = 0
    stored = raw - 1 if fmt == "gptq" else raw
    qweight = og.pack_int_weights(q, bits)
    qzeros = og.pack_zeros(stored, bits)
    scales = np.ones((1, n), dtype=np.float16)
    x = np.zeros((1, k), dtype=np.float16)
    x[0, 0] = 1
    return x, qweight, qzeros, scales, og.default_g_idx(k, 32)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("fmt", ["gptq", "gptq_v2"])
def test_exact_zero_probe(bits, fmt):
    x, qw, qz, sc, g = _probe_layer(bits, fmt)
    y = og.gptq_forward(x, qw, qz, sc, g, bits, checkpoint_format=fmt)[0]
    assert np.all(y[:4] == 0) and np.all(y[4:] == -1)


def test_planted_unmasked_restore_is_caught(monkeypatch):
    """Plant vLLM's recalled unmasked v1 restore (z = Zs + 1) in the oracle:
    the exact probe must fail for the wrapped columns."""
    monkeypatch.setattr(og, "restore_zeros", lambda zs, bits, fmt="gptq": np.asarray(zs) + 1)
    x, qw, qz, sc, g = _probe_layer(4, "gptq")
    y = og.gptq_forward(x, qw, qz, sc, g, 4)[0]
    assert not np.all(y[:4] == 0)


def test_planted_straddle_bug_is_caught(monkeypatch):
    """Plant a 3-bit straddle mistake (upper part taken from the same word):
    the bit-stream brute force must disagree."""
    real = og._slot_layout_3bit

    def broken():
        return [(w, off, 3 if off == 30 else first) for (w, off, first) in real()]

    monkeypatch.setattr(og, "_slot_layout_3bit", broken)
    rng = _rng(3)
    qw = rng.integers(-(2**31), 2**31, size=(3, 2), dtype=np.int64).astype(np.int32)
    codes = og.unpack_int_weights(qw, 3, (2, 32))
    assert codes[0].tolist() != _bitstream_codes(qw[:, 0], 3, 32) or \
        codes[1].tolist() != _bitstream_codes(qw[:, 1], 3, 32)


def test_g_idx_act_order_known_answer():
    """tests/vllm_plugins/test_enable_actorder.py:28-46 restated: g_idx equals
    argsort(perm)//gs; here computed independently by inverting perm by hand."""
    for perm, gs in (([2, 0, 3, 1, 6, 4, 7, 5], 2), ([1, 3, 0, 2], 2)):
        inv = [0] * len(perm)
        for i, p in enumerate(perm):
            inv[p] = i
        assert og.g_idx_from_perm(np.array(perm), gs).tolist() == [v // gs for v in inv]
    assert og.default_g_idx(8, -1).tolist() == [0] * 8
    assert og.default_g_idx(8, 4).tolist() == [0, 0, 0, 0, 1, 1, 1, 1]


def _fp16_rne_exact(value: Fraction) -> np.float16:
    """Nearest fp16 to an exact rational, ties to even, by brute force over
    the two float16 neighbours of a float64 approximation."""
    approx = np.float16(float(value))
    cands = {approx, np.nextafter(approx, np.float16(np.inf)), np.nextafter(approx, np.float16(-np.inf))}
    best = sorted(cands, key=lambda c: (abs(Fraction(float(c)) - value),
                                         int(np.array(c).view(np.uint16)) & 1))
    return best[0]


def test_dequant_single_rounding_fp16_matches_exact_rational():
    rng = _rng(7)
    for bits in BITS:
        s = (np.abs(rng.normal(0, 0.02, 200)) + 1e-3).astype(np.float16)
        q = rng.integers(0, 1 << bits, 200)
        z = rng.integers(0, 1 << bits, 200)
        # N = 200 columns, K = 1, one group
        got = og.round_to(og.dequant_fp32(q[:, None], s[None, :], z[None, :],
                                          np.zeros(1, np.int64)), "fp16")
        for i in range(200):
            exact = Fraction(float(s[i])) * (int(q[i]) - int(z[i]))
            assert got[i, 0] == _fp16_rne_exact(exact), (bits, i)


def test_bf16_rounding_matches_torch():
    torch = pytest.importorskip("torch")
    rng = _rng(8)
    x = rng.normal(0, 3, 4096).astype(np.float32)
    # exact ties: low 16 bits == 0x8000, with both parities of bit 16
    ties = (rng.integers(0x3F000000, 0x42000000, 512).astype(np.uint32) & 0xFFFF0000) | 0x8000
    x = np.concatenate([x, ties.view(np.float32), np.array([0.0, -0.0, 1e-40, 3.4e38], np.float32)])
    want = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(og.f32_to_bf16_bits(x), want)


@pytest.mark.parametrize("bits", BITS)
@pytest.mark.parametrize("act_order", [False, True])
def test_dequant_matches_per_group_loop(bits, act_order):
    """The reference test's own formulation (test_gptq_layer_pack.py:195-199:
    loop over groups, scale*(q - zero)) on natural order, and a per-element
    loop for act-order, agree bit-for-bit with the vectorised oracle."""
    rng = _rng(20 + bits)
    n, k, gs = 32, 256, 64
    q = rng.integers(0, 1 << bits, (n, k)).astype(np.int32)
    zr = rng.integers(0, 1 << bits, (k // gs, n)).astype(np.int32)
    s = (np.abs(rng.normal(0, 0.02, (k // gs, n))) + 1e-3).astype(np.float16)
    if act_order:
        g = og.g_idx_from_perm(rng.permutation(k), gs)
    else:
        g = og.default_g_idx(k, gs)
    qw, qz = og.pack_int_weights(q, bits), og.pack_zeros((zr - 1), bits)
    w = og.dequantize(qw, qz, s, g, bits, "gptq", "fp16")
    ref = np.zeros((n, k), dtype=np.float32)
    for kk in range(k):
        gi = g[kk]
        ref[:, kk] = s[gi].astype(np.float32) * (q[:, kk].astype(np.float32) - zr[gi].astype(np.float32))
    assert np.array_equal(w.view(np.uint16), ref.astype(np.float16).view(np.uint16))


def test_linear_ref_is_fp32_accumulated():
    rng = _rng(9)
    x = rng.normal(size=(3, 64)).astype(np.float16)
    w = rng.normal(size=(5, 64)).astype(np.float16)
    y = og.linear_ref(x, w)
    want = np.array([[sum(float(x[i, j]) * float(w[o, j]) for j in range(64)) for o in range(5)]
                     for i in range(3)], dtype=np.float32)
    assert np.allclose(y, want, rtol=1e-6, atol=1e-6)
