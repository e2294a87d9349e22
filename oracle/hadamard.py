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
- ``fwht_staged`` / ``online_hadamard_rounded``: the same with the rounding
  points of apply_online_hadamard: fp32_had=True runs matmul_hadU_cuda on
  x.float() (transform and division in float32, the product summed exactly
  from the float32 values) and rounds once in ``.to(x_dtype)`` ('fp32');
  fp32_had=False runs it in the activation dtype: the transform rounds every
  butterfly stage with the reference's pure-PyTorch op ('stages'; its
  default install) or once with the fast_hadamard_transform package
  ('once'; sums taken exact), the division by torch.tensor(n).sqrt() (a
  float32 value) rounds, and the H_K matmul (fp32 accumulation, exact here)
  rounds.  Pinned by hand-derived known answers where the three differ and
  by the float64 form within the roundings' bound
  (tests/test_oracle_hadamard.py).
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


def _round(v: np.ndarray, dtype: str) -> np.ndarray:
    """RNE of float values to the activation dtype, returned as float64 values."""
    if dtype == "fp16":
        return np.asarray(v, dtype=np.float64).astype(np.float32).astype(np.float16).astype(np.float64)
    # bf16: round the float32 value (the values here are float32-exact or float32 results)
    u = np.ascontiguousarray(np.asarray(v, dtype=np.float64).astype(np.float32)).view(np.uint32).astype(np.uint64)
    b = ((u + (((u >> 16) & 1) + 0x7FFF)) >> 16).astype(np.uint32) << 16
    return b.view(np.float32).astype(np.float64)


def fwht_staged(x: np.ndarray, dtype: str) -> np.ndarray:
    """hadamard_utils.py:26-44 run in the activation dtype: every stage's sums and differences
    rounded (bit 0 first, as the reference's loop over m = 1, 2, 4, ...)."""
    out = _round(np.asarray(x, dtype=np.float64), dtype)
    n = out.shape[-1]
    m = 1
    while m < n:
        v = out.reshape(*out.shape[:-1], n // (2 * m), 2 * m)
        left, right = v[..., :m].copy(), v[..., m:].copy()
        v[..., :m] = _round(left + right, dtype)
        v[..., m:] = _round(left - right, dtype)
        out = v.reshape(*out.shape[:-1], n)
        m *= 2
    return out


def online_hadamard_rounded(x: np.ndarray, dtype: str, rounding: str = "stages") -> np.ndarray:
    """apply_online_hadamard (rotation.py:100-112 -> hadamard_utils.py:178-199) with its roundings.

    x: activation values [M, n] (exactly representable in ``dtype``, 'fp16' or 'bf16'); rounding:
    'fp32' (fp32_had=True), 'once' (fp32_had=False, fused transform op), 'stages' (fp32_had=False,
    the pure-PyTorch transform).  Returns the output values as float64.
    """
    x = np.asarray(x, dtype=np.float64)
    n = x.shape[-1]
    K = pick_order(n)
    s32 = np.float32(np.sqrt(np.float32(n)))  # torch.tensor(n).sqrt(): float32
    xv = x.reshape(-1, K, n // K)
    if rounding == "fp32":
        u = (fwht(xv).astype(np.float32) / s32).astype(np.float64)
    elif rounding == "once":
        u = _round(_round(fwht(xv), dtype).astype(np.float32) / s32, dtype)
    elif rounding == "stages":
        u = _round(fwht_staged(xv, dtype).astype(np.float32) / s32, dtype)
    else:
        raise ValueError(f"rounding {rounding!r}")
    if K > 1:
        u = np.einsum("ic,mcj->mij", hadamard_block(K).astype(np.float64), u)
    return _round(u, dtype).reshape(x.shape)


def online_hadamard(x: np.ndarray) -> np.ndarray:
    """(H_K (x) H_L) x / sqrt(n) per row of x [M, n], float64."""
    x = np.asarray(x, dtype=np.float64)
    n = x.shape[-1]
    K = pick_order(n)
    u = fwht(x.reshape(-1, K, n // K)) / np.sqrt(n)
    if K > 1:
        u = np.einsum("ic,mcj->mij", hadamard_block(K).astype(np.float64), u)
    return u.reshape(x.shape)
