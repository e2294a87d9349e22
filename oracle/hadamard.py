"""CPU restatement of OneComp's online Hadamard transform (test infrastructure).

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline may use this
module, as the checker.  The product path is onecompression_amd/csrc/hadamard.hip.

- ``pick_order``: the block order search of hadamard_utils.py:79-175 (the
  largest listed K dividing n with n / K a power of two; n itself a power of
  two gives K = 1).
- ``hadamard_block``: the K x K matrices, built from the classical
  constructions (Paley I, Paley II, Sylvester doubling, the Williamson array
  for 52, 100, 156, 172) instead of the reference's literal tables.  Pinned:
  tests compare the SHA-256 of each construction with
  tests/golden/hadamard_digests.json, written from the reference's tables.
- ``fwht``: the unnormalised natural-order transform of
  hadamard_utils.py:26-44 (butterfly (a, b) -> (a + b, a - b) on blocks of
  2m).  Pinned by the closed form H[i, j] = (-1)^popcount(i & j).
- ``online_hadamard``: matmul_hadU_cuda (hadamard_utils.py:178-199) as used by
  apply_online_hadamard (vllm_plugins/utils/rotation.py:100-112), in float64.
"""

from __future__ import annotations

import numpy as np

# (K, construction, q) in the reference's search order (hadamard_utils.py:93-172)
ORDERS = [(172, "williamson", 43), (156, "williamson", 39), (140, "paley1", 139), (108, "paley1", 107),
          (100, "williamson", 25), (76, "paley2", 37), (68, "paley1", 67), (60, "paley1", 59),
          (52, "williamson", 13), (44, "paley1", 43), (40, "double", 20), (36, "paley2", 17),
          (28, "paley2", 13), (20, "paley1", 19), (12, "paley1", 11)]

# Williamson generators per q: the first (q + 1) / 2 signs of the first rows of the symmetric
# circulants A, B, C, D (the data that singles out the reference's matrices of orders 4q).
WILLIAMSON = {
    13: ("+-+--++", "+---+++", "++-+--+", "+----+-"),
    25: ("+-++++----++-", "+++-+++---+-+", "+-++-+++-++--", "+--++-+-+----"),
    39: ("+++--+-+-----+--++--", "++++---+--++----+-+-", "+++--++-+---+-+--+--", "+---++-+-+-----+++-+"),
    43: ("+---++--++++-+-+++-++-", "++-++++++----+-+--++-+", "+++-+-++--+-+-++++-+--", "++---++++-+--+--++----"),
}


def is_pow2(n: int) -> bool:
    return n > 0 and (n & (n - 1)) == 0


def pick_order(n: int) -> int:
    """Block order for dimension n; raises like the reference's asserts."""
    for K, _, _ in ORDERS:
        if n % K == 0:
            if not is_pow2(n // K):
                raise ValueError(f"n={n}: n/{K} is not a power of 2")
            return K
    if not is_pow2(n):
        raise ValueError(f"n={n} is not a power of 2")
    return 1


def _chi(q: int) -> np.ndarray:
    """Quadratic character of Z/q as a table chi[a], a in [0, q)."""
    c = -np.ones(q, dtype=np.int64)
    c[0] = 0
    for x in range(1, q):
        c[(x * x) % q] = 1
    return c


def paley1(q: int) -> np.ndarray:
    """Order q + 1 (q prime, q = 3 mod 4): I + [[0, -1^T], [1, chi(a - b)]]."""
    chi = _chi(q)
    a = np.arange(q)
    S = np.zeros((q + 1, q + 1), dtype=np.int64)
    S[0, 1:] = -1
    S[1:, 0] = 1
    S[1:, 1:] = chi[(a[:, None] - a[None, :]) % q]
    return S + np.eye(q + 1, dtype=np.int64)


def paley2(q: int) -> np.ndarray:
    """Order 2(q + 1) (q prime, q = 1 mod 4): A (x) C + B (x) I."""
    chi = _chi(q)
    a = np.arange(q)
    C = np.zeros((q + 1, q + 1), dtype=np.int64)
    C[0, 1:] = 1
    C[1:, 0] = 1
    C[1:, 1:] = chi[(a[None, :] - a[:, None]) % q]
    A = np.array([[1, 1], [1, -1]])
    B = np.array([[1, -1], [-1, -1]])
    return np.kron(A, C) + np.kron(B, np.eye(q + 1, dtype=np.int64))


def symmetric_circulant(half: str, q: int) -> np.ndarray:
    """q x q circulant X[i, j] = x[(j - i) mod q] with x[j] = x[q - j] given by its first half."""
    h = np.array([1 if c == "+" else -1 for c in half], dtype=np.int64)
    x = np.concatenate([h, h[1:q - len(h) + 1][::-1]])
    idx = (np.arange(q)[None, :] - np.arange(q)[:, None]) % q
    return x[idx]


def williamson(q: int) -> np.ndarray:
    """Order 4q: [[A, B, C, D], [-B, A, -D, C], [-C, D, A, -B], [-D, -C, B, A]]."""
    A, B, C, D = (symmetric_circulant(h, q) for h in WILLIAMSON[q])
    return np.block([[A, B, C, D], [-B, A, -D, C], [-C, D, A, -B], [-D, -C, B, A]])


def hadamard_block(K: int) -> np.ndarray:
    if K == 1:
        return np.ones((1, 1), dtype=np.int64)
    for k, how, q in ORDERS:
        if k != K:
            continue
        if how == "paley1":
            return paley1(q)
        if how == "paley2":
            return paley2(q)
        if how == "double":
            return np.kron(np.array([[1, 1], [1, -1]]), hadamard_block(q))
        if how == "williamson":
            return williamson(q)
        raise NotImplementedError(f"Hadamard order {K} is not constructed")
    raise ValueError(f"no Hadamard order {K}")


def fwht(x: np.ndarray) -> np.ndarray:
    """Unnormalised natural-order Walsh-Hadamard transform along the last axis."""
    out = np.array(x, dtype=np.float64, copy=True)
    n = out.shape[-1]
    m = 1
    while m < n:
        v = out.reshape(*out.shape[:-1], n // (2 * m), 2 * m)
        left, right = v[..., :m].copy(), v[..., m:].copy()
        v[..., :m] = left + right
        v[..., m:] = left - right
        out = v.reshape(*out.shape[:-1], n)
        m *= 2
    return out


def online_hadamard(x: np.ndarray) -> np.ndarray:
    """(H_K (x) H_L) x / sqrt(n) per row of x [M, n], float64."""
    x = np.asarray(x, dtype=np.float64)
    n = x.shape[-1]
    K = pick_order(n)
    u = fwht(x.reshape(-1, K, n // K)) / np.sqrt(n)
    if K > 1:
        u = np.einsum("ic,mcj->mij", hadamard_block(K).astype(np.float64), u)
    return u.reshape(x.shape)
