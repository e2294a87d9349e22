"""CPU restatement of OneComp's quantized-linear path: TEST INFRASTRUCTURE ONLY.

This package is the checker, never the product.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it.  The HIP library in ``onecompression_amd`` never routes through it
and fails loudly when its native extension is missing.

Modules:

- :mod:`oracle.gptq` -- AutoGPTQ bit layout (2/3/4/8-bit pack/unpack along K
  and along N), the v1/v2 zero restore, ``g_idx`` construction and the
  single-rounding dequantisation ``W = RNE(scale * (q - zero))``.
- :mod:`oracle.dbf` -- DBF/MDBF sign packing (uint8, MSB first, flat
  row-major, padding = +1), the DBF rank formula and the 5-stage / P-path
  forwards.

Every function cites the reference file:line it restates.  Each function is
pinned by tests in ``tests/test_oracle_*.py`` against the reference's own
known-answer tests, an independent brute-force restatement, or a closed form
(see the per-function docstrings for which).
"""
