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


def _per_scale_forward(x, path):
    """Independent float64 evaluation of the reference's per-scale form of one MDBF path
    (mdbf_layer.py:307-336): u = sum_k ((x * B_amp[:, k]) @ S_B^T) * Q_V[:, k], then
    y = sum_k ((u * Q_U[:, k]) @ S_A^T) * A_amp[:, k].  No factor matrix is formed."""
    sa = od.unpack_binary_factor(path["A_sign_packed"], path["A_shape"]).astype(np.float64)
    sb = od.unpack_binary_factor(path["B_sign_packed"], path["B_shape"]).astype(np.float64)
    f = lambda a: np.asarray(a, np.float64)  # noqa: E731
    a_amp, b_amp, qu, qv = f(path["A_amp"]), f(path["B_amp"]), f(path["Q_U_amp"]), f(path["Q_V_amp"])
    xf = f(x)
    u = sum(((xf * b_amp[:, k]) @ sb.T) * qv[:, k] for k in range(b_amp.shape[1]))
    return sum(((u * qu[:, k]) @ sa.T) * a_amp[:, k] for k in range(a_amp.shape[1]))


def _mdbf_path(n, r, m, l, seed):
    rng = np.random.default_rng(seed)
    amp = lambda d: (np.abs(rng.normal(0, 0.3, (d, l))) + 0.05).astype(np.float32)  # noqa: E731
    return dict(A_sign_packed=od.pack_binary(rng.choice([-1, 1], size=(n, r))), A_shape=(n, r),
                B_sign_packed=od.pack_binary(rng.choice([-1, 1], size=(r, m))), B_shape=(r, m),
                A_amp=amp(n), B_amp=amp(m), Q_U_amp=amp(r), Q_V_amp=amp(r))


@pytest.mark.parametrize("l", [2, 3])
def test_mdbf_multi_scale_matches_per_scale_form(l):
    """The oracle's materialised-factor forward (mdbf_layer.py:278-290, :338-344) against the
    reference's own per-scale reformulation (:307-336), evaluated independently in float64.
    In fp32 mode (no 16-bit rounding of the amp products) the two agree to fp32 precision; in
    fp16 mode within the per-element rounding of the factors.  Two paths check the P-sum
    (:412-420)."""
    n, r, m = 40, 24, 56
    paths = [_mdbf_path(n, r, m, l, 10 * l + p) for p in range(2)]
    x = np.random.default_rng(l).normal(size=(5, m)).astype(np.float32)
    want = sum(_per_scale_forward(x, p) for p in paths)
    got = od.mdbf_forward(x, paths, dtype="fp32")
    assert np.max(np.abs(got - want)) / np.max(np.abs(want)) < 1e-5
    x16 = x.astype(np.float16)
    paths16 = [{k: (v.astype(np.float16) if k.endswith("amp") else v) for k, v in p.items()} for p in paths]
    want16 = sum(_per_scale_forward(x16, p) for p in paths16)
    got16 = od.mdbf_forward(x16, paths16, dtype="fp16")
    assert np.max(np.abs(got16 - want16)) / np.max(np.abs(want16)) < 1e-2


def test_mdbf_planted_qu_qv_swap_is_caught(monkeypatch):
    """A planted Q_U <-> Q_V swap in the oracle's factor construction (possible only for l > 1
    to matter) must fail the per-scale comparison."""
    real = od.mdbf_path_factors

    def swapped(a_packed, a_shape, b_packed, b_shape, a_amp, b_amp, qu_amp, qv_amp, dtype="fp16"):
        return real(a_packed, a_shape, b_packed, b_shape, a_amp, b_amp, qv_amp, qu_amp, dtype)

    n, r, m, l = 40, 24, 56, 2
    paths = [_mdbf_path(n, r, m, l, 77)]
    x = np.random.default_rng(78).normal(size=(5, m)).astype(np.float32)
    want = _per_scale_forward(x, paths[0])
    assert np.max(np.abs(od.mdbf_forward(x, paths, dtype="fp32") - want)) / np.max(np.abs(want)) < 1e-5
    monkeypatch.setattr(od, "mdbf_path_factors", swapped)
    bad = od.mdbf_forward(x, paths, dtype="fp32")
    assert np.max(np.abs(bad - want)) / np.max(np.abs(want)) > 1e-2
