"""The C-ABI library loads and exports every symbol include/onecomp_amd.h declares (CPU only)."""

import ctypes
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "onecomp_amd.h")


def _declared():
    src = open(HEADER).read()
    src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
    return sorted(set(re.findall(r"\b(oc_[a-z0-9_]+)\s*\(", src)))


def test_header_matches_binding_table():
    from onecompression_amd import _native

    assert _declared() == sorted(_native.SIGNATURES)


def test_library_exports_every_declared_symbol():
    from onecompression_amd import _native

    if not os.path.exists(_native.LIB_PATH):
        pytest.fail("library not built: run python -m onecompression_amd.build")
    lib = ctypes.CDLL(_native.LIB_PATH)
    missing = [name for name in _declared() if not hasattr(lib, name)]
    assert not missing, missing


def test_host_only_entry_points():
    from onecompression_amd import _native, ops

    lib = _native.load()
    assert lib.oc_abi_version() == _native.ABI_VERSION
    nbytes, kp, np_ = ops.gptq_layout(4096, 4096, 4)
    assert (nbytes, kp, np_) == (4096 * 4096 // 2, 4096, 4096)
    nbytes, kp, np_ = ops.gptq_layout(14336, 4096, 2)
    assert (nbytes, kp) == (14336 * 4096 // 4, 14336)
    nbytes, kp, _ = ops.gptq_layout(4096, 14336, 3)
    assert nbytes == 4096 * 14336 * 3 // 8 and kp == 4096
    nbytes, kp, np_ = ops.gptq_layout(4160, 100, 8)
    assert kp == 4224 and np_ == 112 and nbytes == 4224 * 112
    with pytest.raises(_native.OCError, match="UNSUPPORTED"):
        ops.gptq_layout(4096, 4096, 5)
    assert "bits=5" in _native.last_error()
