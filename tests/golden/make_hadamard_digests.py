"""Digests of the reference's Hadamard blocks (run in the build container only).

Reads onecomp/pre_process/hadamard_utils.py of the reference as text (the
matrices are literal tables there), and records for every order K the
SHA-256 of the K x K matrix as int8 row-major bytes.  Only the digests are
committed: the tests compare oracle/hadamard.py's constructions with them.
"""

import hashlib
import json
import os
import re
import sys

import numpy as np

REF = "/root/reference/onecomp/pre_process/hadamard_utils.py"
OUT = os.path.join(os.path.dirname(os.path.abspath(__file__)), "hadamard_digests.json")


def parse(src, K):
    i = src.index(f"def get_had{K}():")
    j = src.index("torch.FloatTensor(", i)
    k = src.index("\n    )", j)
    rows = re.findall(r"\[([^\[\]]*)\]", src[j + len("torch.FloatTensor("):k])
    return np.array([[int(float(v)) for v in r.replace("\n", " ").split(",") if v.strip()] for r in rows],
                    dtype=np.int8)


def main():
    if not os.path.exists(REF):
        sys.exit(f"{REF} not found (this script runs where the reference is mounted)")
    src = open(REF).read()
    orders = sorted(int(k) for k in re.findall(r"def get_had(\d+)\(\):", src))
    out = {"source": "onecomp/pre_process/hadamard_utils.py (get_had<K>), int8 row-major SHA-256",
           "digests": {}}
    for K in orders:
        H = parse(src, K)
        assert H.shape == (K, K) and np.array_equal(H.astype(np.int64) @ H.T.astype(np.int64), K * np.eye(K))
        out["digests"][str(K)] = hashlib.sha256(np.ascontiguousarray(H).tobytes()).hexdigest()
    with open(OUT, "w") as f:
        json.dump(out, f, indent=1)
    print(f"wrote {len(orders)} digests to {OUT}")


if __name__ == "__main__":
    main()
