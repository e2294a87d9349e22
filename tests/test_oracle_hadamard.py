"""The online-Hadamard oracle and the C ABI's host-side block construction."""

import hashlib
import json
import os

import numpy as np
import pytest

from oracle import hadamard as oh

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "hadamard_digests.json")
BUILT = [K for K, how, _ in oh.ORDERS if how is not None]


def _digest(H):
    return hashlib.sha256(np.ascontiguousarray(np.asarray(H, dtype=np.int8)).tobytes()).hexdigest()


@pytest.mark.parametrize("K", BUILT)
def test_blocks_match_reference_tables(K):
    """The constructions reproduce get_had<K> of hadamard_utils.py bit for bit (digests of the tables)."""
    with open(GOLDEN) as f:
        digests = json.load(f)["digests"]
    H = oh.hadamard_block(K)
    assert H.shape == (K, K)
    assert np.array_equal(H @ H.T, K * np.eye(K, dtype=np.int64))
    assert _digest(H) == digests[str(K)]


def test_planted_mistake_is_caught():
    """Jacobsthal sign flipped (chi(b - a) instead of chi(a - b)): still Hadamard, wrong digest."""
    with open(GOLDEN) as f:
        digests = json.load(f)["digests"]
    chi = oh._chi(11)
    a = np.arange(11)
    S = np.zeros((12, 12), dtype=np.int64)
    S[0, 1:], S[1:, 0] = -1, 1
    S[1:, 1:] = chi[(a[None, :] - a[:, None]) % 11]
    H = S + np.eye(12, dtype=np.int64)
    assert np.array_equal(H @ H.T, 12 * np.eye(12, dtype=np.int64))
    assert _digest(H) != digests["12"]


def test_every_reference_order_is_built():
    with open(GOLDEN) as f:
        digests = json.load(f)["digests"]
    assert sorted(BUILT) == sorted(int(k) for k in digests)


def test_williamson_planted_mistake_is_caught():
    """The Williamson array with the roles of B and C exchanged in the second block row is no
    longer the reference's matrix (and no longer orthogonal)."""
    with open(GOLDEN) as f:
        digests = json.load(f)["digests"]
    q = 13
    A, B, C, D = (oh.symmetric_circulant(h, q) for h in oh.WILLIAMSON[q])
    H = np.block([[A, B, C, D], [-C, A, -D, B], [-B, D, A, -C], [-D, -C, B, A]])
    assert _digest(H) != digests["52"]
    good = oh.williamson(q)
    assert np.array_equal(good @ good.T, 52 * np.eye(52, dtype=np.int64))


def test_symmetric_circulant_closed_form():
    X = oh.symmetric_circulant("+--+", 7)
    assert np.array_equal(X, X.T)
    assert X[0].tolist() == [1, -1, -1, 1, 1, -1, -1]
    assert all(np.array_equal(np.roll(X[0], i), X[i]) for i in range(7))


def test_pick_order():
    assert oh.pick_order(14336) == 28      # Llama-3-8B intermediate
    assert oh.pick_order(12288) == 12      # Qwen3-8B intermediate
    assert oh.pick_order(17408) == 68      # Qwen3-14B intermediate
    assert oh.pick_order(11008) == 172     # Llama-2-7B intermediate
    assert oh.pick_order(4096) == 1
    for bad in (3 * 28 * 8, 105, 1000):
        with pytest.raises(ValueError):
            oh.pick_order(bad)


def test_fwht_closed_form():
    n = 64
    i = np.arange(n)
    sylvester = (-1.0) ** np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    assert np.array_equal(oh.fwht(np.eye(n)), sylvester)
    assert np.array_equal(oh.fwht(np.eye(n)[0]), np.ones(n))


@pytest.mark.parametrize("n", [16, 24, 56, 80])
def test_online_hadamard_is_the_normalised_kronecker_product(n):
    T = oh.online_hadamard(np.eye(n))  # row m = transform of e_m
    K = oh.pick_order(n)
    L = n // K
    i = np.arange(L)
    HL = (-1.0) ** np.vectorize(lambda v: bin(v).count("1"))(i[:, None] & i[None, :])
    expect = np.kron(oh.hadamard_block(K).astype(np.float64), HL) / np.sqrt(n)
    assert np.allclose(T, expect.T, atol=1e-12)
    assert np.allclose(T @ T.T, np.eye(n), atol=1e-12)


def test_c_abi_blocks_and_orders_match_oracle():
    """Host-only entry points of the library (no GPU needed)."""
    import ctypes

    from onecompression_amd import _native as N

    lib = N.load()
    for K in BUILT + [1]:
        buf = (ctypes.c_int8 * (K * K))()
        assert lib.oc_hadamard_block(K, buf) == 0
        assert np.array_equal(np.array(list(buf), dtype=np.int64).reshape(K, K), oh.hadamard_block(K))
    for K in (24, 48, 88):
        buf = (ctypes.c_int8 * (K * K))()
        assert lib.oc_hadamard_block(K, buf) == N.OC_ERR_UNSUPPORTED
    for n in (14336, 12288, 17408, 11008, 4096, 640, 25600, 6656, 9984):
        assert lib.oc_hadamard_order(n) == oh.pick_order(n)
    assert lib.oc_hadamard_order(1000) == 0


# The reference's rounding points (rotation.py:100-112 -> hadamard_utils.py:26-44, :178-199), pinned
# by answers derived by hand: fp16 [2048, 1, 1, 1] (n = 4, K = 1, sqrt = 2).  Pure-PyTorch stages:
# bit 0: [2048 + 1 -> 2048 (tie to even), 2047, 2, 0]; bit 1: [2050, 2047, 2046, 2047]; / 2.
# Fused op: the exact 2051 rounds to 2052, / 2 = 1026.  fp32: 2051 / 2 = 1025.5 -> 1026 (tie, even).
def test_rounded_known_answers_fp16():
    x = np.array([[2048, 1, 1, 1]], dtype=np.float64)
    assert oh.online_hadamard_rounded(x, "fp16", "stages").tolist() == [[1025, 1023.5, 1023, 1023.5]]
    assert oh.online_hadamard_rounded(x, "fp16", "once").tolist() == [[1026, 1023.5, 1023.5, 1023.5]]
    assert oh.online_hadamard_rounded(x, "fp16", "fp32").tolist() == [[1026, 1023.5, 1023.5, 1023.5]]


def test_rounded_known_answers_bf16():
    # bf16 spacing 2 at 256: 256 + 1 -> 256; the exact 259 -> 260; 259 / 2 = 129.5 -> 130
    x = np.array([[256, 1, 1, 1]], dtype=np.float64)
    assert oh.online_hadamard_rounded(x, "bf16", "stages").tolist() == [[129, 127.5, 127, 127.5]]
    assert oh.online_hadamard_rounded(x, "bf16", "once").tolist() == [[130, 127.5, 127.5, 127.5]]
    assert oh.online_hadamard_rounded(x, "bf16", "fp32").tolist() == [[130, 127.5, 127.5, 127.5]]


def test_rounded_stage_order_planted():
    """Stages taken high bit first (a plausible mistake) change the known answer above."""
    x = np.array([[2048, 1, 1, 1]], dtype=np.float64)
    v = x.copy()
    for m in (2, 1):  # reversed
        w = v.reshape(1, 4 // (2 * m), 2 * m)
        left, right = w[..., :m].copy(), w[..., m:].copy()
        w[..., :m] = oh._round(left + right, "fp16")
        w[..., m:] = oh._round(left - right, "fp16")
        v = w.reshape(1, 4)
    wrong = oh._round(v.astype(np.float32) / np.float32(2), "fp16")
    assert wrong.tolist() != oh.online_hadamard_rounded(x, "fp16", "stages").tolist()


@pytest.mark.parametrize("n", [4096, 14336, 12288, 11008])
@pytest.mark.parametrize("rounding,tol", [("fp32", 1e-3), ("once", 2e-3), ("stages", 1e-2)])
def test_rounded_near_float64(n, rounding, tol):
    rng = np.random.default_rng(n)
    x = rng.standard_normal((2, n)).astype(np.float16).astype(np.float64)
    ref = oh.online_hadamard(x)
    got = oh.online_hadamard_rounded(x, "fp16", rounding)
    assert np.max(np.abs(got - ref)) / np.max(np.abs(ref)) <= tol
