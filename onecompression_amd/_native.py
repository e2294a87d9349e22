"""ctypes binding of the C ABI in ``include/onecomp_amd.h`` (``lib/liboc_quant.so``).

The library is loaded after ``import torch`` so that it shares the HIP runtime
torch already loaded (both use the soname ``libamdhip64.so.7``).  There is no
fallback: if the library is missing, every entry point raises.
"""

from __future__ import annotations

import ctypes
import os
import threading

_PKG = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("ONECOMP_AMD_LIB", os.path.join(_PKG, "lib", "liboc_quant.so"))

c_int, c_size_t, c_void_p = ctypes.c_int, ctypes.c_size_t, ctypes.c_void_p
c_char_p = ctypes.c_char_p
P = ctypes.c_void_p  # every device pointer travels as an untyped address
c_int_p = ctypes.POINTER(ctypes.c_int)
c_size_t_p = ctypes.POINTER(ctypes.c_size_t)

# name -> (restype, argtypes); mirrors include/onecomp_amd.h one for one
SIGNATURES = {
    "oc_abi_version": (c_int, []),
    "oc_last_error": (c_char_p, []),
    "oc_set_plan_override": (c_int, [c_char_p, c_int]),
    "oc_clear_plan_overrides": (None, []),
    "oc_plan_generation": (c_int, []),
    "oc_gptq_unpack_codes": (c_int, [P, c_int, c_int, c_int, P, P]),
    "oc_gptq_unpack_zeros": (c_int, [P, c_int, c_int, c_int, c_int, P, P]),
    "oc_gptq_dequant": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, c_int, P, P]),
    "oc_gptq_layout": (c_int, [c_int, c_int, c_int, c_size_t_p, c_int_p, c_int_p]),
    "oc_gptq_prepare": (c_int, [P, P, P, P, c_int, c_int, c_int, c_int, c_int, c_int, P, P, P,
                                c_int_p, P]),
    "oc_gptq_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int, c_int]),
    "oc_gptq_describe_plan": (c_int, [c_int, c_int, c_int, c_int, c_int, c_int, c_char_p, c_int]),
    "oc_gptq_gemm": (c_int, [P, c_int, c_int, c_int, P, P, P, c_int, c_int, c_int, P, P, P,
                             c_size_t, P]),
    "oc_gptq_gemm_noalloc": (c_int, [P, c_int, c_int, c_int, P, P, P, c_int, c_int, c_int, P, P, P]),
    "oc_gptq_noalloc_scratch_bytes": (c_size_t, []),
    "oc_gptq_grouped_workspace_bytes": (c_size_t, [P, c_int, c_int, c_int]),
    "oc_gptq_gemm_grouped": (c_int, [P, c_int, c_int, P, c_int, c_int, P, c_int, P, c_size_t, P]),
    "oc_moe_workspace_bytes": (c_size_t, [c_int, c_int, c_int, c_int, c_int]),
    "oc_moe_gptq_forward": (c_int, [P, c_int, c_int, c_int, c_int, c_int, P, P, P, c_size_t, P, c_size_t,
                                    P, P, c_size_t, P, c_size_t, P, P, P, c_int, c_int, c_int, ctypes.c_float,
                                    ctypes.c_float, c_int, P, P, c_size_t, P]),
    "oc_dbf_layout": (c_int, [c_int, c_int, c_size_t_p, c_int_p, c_int_p]),
    "oc_dbf_unpack_signs": (c_int, [P, c_int, c_int, P, P]),
    "oc_dbf_prepare": (c_int, [P, c_int, c_int, P, P]),
    "oc_sign_workspace_bytes": (c_size_t, [P, c_int, c_int, c_int]),
    "oc_hadamard_order": (c_int, [c_int]),
    "oc_hadamard_block": (c_int, [c_int, P]),
    "oc_hadamard": (c_int, [P, c_int, c_int, c_int, P, c_int, c_int, c_int, P, c_int, P]),
    "oc_sign_gemm": (c_int, [P, c_int, c_int, c_int, c_int, P, P, c_int, c_int, P, c_size_t, P]),
    "oc_sign_batch_workspace_bytes": (c_size_t, [P, c_int, c_int, c_int]),
    "oc_sign_gemm_batch": (c_int, [P, c_int, c_int, c_int, c_int, P, c_int, c_int, P, c_size_t, P]),
}

ABI_VERSION = 7
OC_DTYPE_F16, OC_DTYPE_BF16 = 0, 1
OC_HAD_ROUND_FP32, OC_HAD_ROUND_ONCE, OC_HAD_ROUND_STAGES = 0, 1, 2
OC_ZERO_RAW, OC_ZERO_V1, OC_ZERO_V2 = 0, 1, 2
ERR_NAMES = {-1: "INVALID", -2: "UNSUPPORTED", -3: "SHAPE", -4: "HIP", -5: "WORKSPACE", -6: "GIDX"}
OC_ERR_INVALID, OC_ERR_UNSUPPORTED, OC_ERR_SHAPE, OC_ERR_HIP, OC_ERR_WORKSPACE, OC_ERR_GIDX = -1, -2, -3, -4, -5, -6


class OCError(RuntimeError):
    """A C-ABI call returned a negative status."""

    def __init__(self, code: int, fn: str, msg: str):
        super().__init__(f"{fn} failed with OC_ERR_{ERR_NAMES.get(code, code)}: {msg}")
        self.code = code


_lock = threading.Lock()
_lib = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    """Load the library (no GPU needed) and bind every declared symbol."""
    global _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not os.path.exists(path):
            raise RuntimeError(
                f"onecomp-amd native library not found at {path}; build it with "
                "`python -m onecompression_amd.build` (there is no CPU fallback)"
            )
        import torch  # noqa: F401  -- ensures torch's HIP runtime is the one in the process

        lib = ctypes.CDLL(path, mode=ctypes.RTLD_GLOBAL)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype, fn.argtypes = res, args
        if lib.oc_abi_version() != ABI_VERSION:
            raise RuntimeError(f"ABI mismatch: library {lib.oc_abi_version()} != {ABI_VERSION}")
        _lib = lib
        return lib


def call(name: str, *args) -> int:
    """Call a status-returning entry point and raise OCError on failure."""
    lib = load()
    rc = getattr(lib, name)(*args)
    if rc != 0:
        raise OCError(rc, name, lib.oc_last_error().decode(errors="replace"))
    return rc


def set_plan_override(name: str, value: int) -> None:
    """Pin one launch-plan knob (an ``OC_*`` name) until :func:`clear_plan_overrides` (tests)."""
    call("oc_set_plan_override", name.encode(), int(value))


def clear_plan_overrides() -> None:
    load().oc_clear_plan_overrides()


def plan_generation() -> int:
    """Changes whenever an override is set or cleared (workspace sizes may change with it)."""
    return load().oc_plan_generation()


def describe_gptq_plan(m: int, k: int, n: int, bits: int, group_size: int, has_perm: bool = False) -> str:
    """The launches oc_gptq_gemm makes for this call, as text (host only)."""
    buf = ctypes.create_string_buffer(256)
    call("oc_gptq_describe_plan", m, k, n, bits, group_size, int(has_perm), buf, 256)
    return buf.value.decode()


def last_error() -> str:
    return load().oc_last_error().decode(errors="replace")
