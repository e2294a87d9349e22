"""Pins for the DBF / MDBF oracle (CPU only)."""

import numpy as np
import pytest

from oracle import dbf as od


def test_unpack_known_answers():
    """tests/vllm_plugins/dbf/test_dbf_naive.py:28-56."""
    assert od.unpack_binary_factor(np.array([0b10101010], np.uint8), (1, 8)).tolist() == \
        [[1, -1, 1, -1, 1, -1, 1, -1]]
    got = od.unpack_binary_factor(np.array([0b11001100, 0b00110011], np.uint8), (2, 8))
    assert got.tolist() == [[1, 1, -1, -1, 1, 1, -1, -1], [-1, -1, 1, 1, -1, -1, 1, 1]]


def test_sign_matmul_known_answer():
    """test_dbf_naive.py:110-151: 2x8 signs from [0b10101010, 0b01010101]
    times [[1..8],[8..1]] gives [[-4, 4], [4, -4]]."""
    s = od.unpack_binary_factor(np.array([0b10101010, 0b01010101], np.uint8), (2, 8))
    x = np.array([[1, 2, 3, 4, 5, 6, 7, 8], [8, 7, 6, 5, 4, 3, 2, 1]], np.float64)
    assert (x @ s.T).tolist() == [[-4, 4], [4, -4]]


def test_planted_lsb_first_is_caught(monkeypatch):
    def lsb_first(packed):
        p = np.asarray(packed, np.uint8)
        bits = np.stack([(p >> i) & 1 for i in range(8)], 1).astype(np.int8)
        return bits.reshape(-1) * 2 - 1

    monkeypatch.setattr(od, "unpack_binary", lsb_first)
    got = od.unpack_binary_factor(np.array([0b11001100, 0b00110011], np.uint8), (2, 8))
    assert got.tolist() != [[1, 1, -1, -1, 1, 1, -1, -1], [-1, -1, 1, 1, -1, -1, 1, 1]]


@pytest.mark.parametrize("shape", [(8, 8), (5, 7), (3, 1), (1, 9), (13, 11), (7, 3185 % 64 + 1)])
def test_pack_round_trip_odd_shapes(shape):
    """test_dbf_layer_pack.py:43-56: bit-exact round trip, unaligned rows."""
    rng = np.random.default_rng(shape[0] * 100 + shape[1])
    m = rng.choice([-1, 1], size=shape).astype(np.int8)
    p = od.pack_binary(m)
    assert p.dtype == np.uint8 and p.size == (m.size + 7) // 8
    assert np.array_equal(od.unpack_binary_factor(p, shape), m)
    # padding bits are +1 (dbf_layer.py:36-40)
    pad = (-m.size) % 8
    if pad:
        assert int(p[-1]) & ((1 << pad) - 1) == (1 << pad) - 1


def test_rank_formula():
    """vllm_plugin.py:81-83: int() truncation, so 4096<->14336 gives 3185."""
    assert od.mid_features(1.0, 4096, 14336) == 3185
    assert od.mid_features(1.0, 14336, 4096) == 3185
    assert od.mid_features(1.0, 4096, 4096) == 2048
    assert od.mid_features(8.0, 16, 16) == 16  # clipped at min(K, N)


def test_part_layout_offsets():
    lay = od.part_layout(1.0, 64, [32, 16, 16])
    assert lay["mid_sizes"] == [21, 12, 12]
    assert lay["bp1_sizes"] == [(21 * 64 + 7) // 8, 96, 96]
    assert lay["bp3_sizes"] == [(32 * 21 + 7) // 8, (16 * 12 + 7) // 8, 24]
    assert lay["bp1_offsets"] == [0, 168, 264]


def _factors(k, n, seed):
    rng = np.random.default_rng(seed)
    r = od.mid_features(1.0, k, n)
    s2m = rng.choice([-1, 1], size=(r, k))
    s1m = rng.choice([-1, 1], size=(n, r))
    s0 = (np.abs(rng.normal(0, 0.05, k)) + 1e-3).astype(np.float16)
    s2 = (np.abs(rng.normal(0, 0.05, r)) + 1e-3).astype(np.float16)
    s4 = (np.abs(rng.normal(0, 0.05, n)) + 1e-3).astype(np.float16)
    return r, od.pack_binary(s2m), od.pack_binary(s1m), s0, s2, s4, s2m, s1m


def test_dbf_forward_matches_dense_weight():
    """Factorised 5-stage forward == x @ W^T with W formed densely from the
    unpacked factors (closed form of dequantize.py:40-77)."""
    k, n = 96, 40
    r, bp1, bp3, s0, s2, s4, s2m, s1m = _factors(k, n, 1)
    x = np.random.default_rng(2).normal(size=(3, k)).astype(np.float16)
    y = od.dbf_forward(x, s0, bp1, s2, bp3, s4, k, r, n)
    w = (s4.astype(np.float64)[:, None] * (s1m @ (s2.astype(np.float64)[:, None] * s2m))
         * s0.astype(np.float64)[None, :])
    assert np.allclose(y, x.astype(np.float64) @ w.T, rtol=1e-6, atol=1e-9)
    ys = od.dbf_forward(x, s0, bp1, s2, bp3, s4, k, r, n, staged=True)
    assert np.max(np.abs(ys - y)) / np.max(np.abs(y)) < 1e-2


def test_mdbf_l1_equals_dbf_closed_form():
    """An l=1 MDBF path is DBF with a=A_amp, m=Q_U*Q_V, b=B_amp (up to the
    per-element rounding of the amp products, mdbf_layer.py:284-288)."""
    k, n = 64, 48
    r, bp1, bp3, s0, s2, s4, s2m, s1m = _factors(k, n, 3)
    path = dict(A_sign_packed=bp3, A_shape=(n, r), B_sign_packed=bp1, B_shape=(r, k),
                A_amp=s4.reshape(n, 1), B_amp=s0.reshape(k, 1),
                Q_U_amp=s2.reshape(r, 1), Q_V_amp=np.ones((r, 1), np.float16))
    x = np.random.default_rng(4).normal(size=(2, k)).astype(np.float16)
    y = od.mdbf_forward(x, [path, path])
    yd = 2 * od.dbf_forward(x, s0, bp1, s2, bp3, s4, k, r, n)
    assert np.max(np.abs(y - yd)) / np.max(np.abs(yd)) < 1e-2
