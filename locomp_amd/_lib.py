"""ctypes binding of ``_liblocomp_amd.so`` (declared in include/locomp_amd.h).

The reference binds one generated ``locomp_launch_<name>`` per kernel with
ctypes (locomp/api.py:949-990); this module binds the hand-written library
once.  There is no fallback: if the library is missing, every launch raises.
"""

from __future__ import annotations

import ctypes
import os
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "_liblocomp_amd.so"

ABI_VERSION = 5

# dtype codes (LQ_F32 / LQ_F16 / LQ_BF16)
F32, F16, BF16 = 0, 1, 2
# error codes
OK, ERR_SHAPE, ERR_DTYPE, ERR_NULL, ERR_POLICY, ERR_SCRATCH, ERR_NAME = 0, -1, -2, -3, -4, -5, -6
# kernel policies
POLICY_AUTO, POLICY_GENERIC = 0, 1
# quantizer variants (LQ_QUANT_EX38 / LQ_QUANT_EX52)
QUANT_EX38, QUANT_EX52 = 0, 1

_i64 = ctypes.c_int64
_int = ctypes.c_int
_vp = ctypes.c_void_p

# name -> argtypes, in header order
SIGNATURES = {
    "locomp_amd_abi_version": [],
    "locomp_amd_strerror": [_int],
    "locomp_amd_set_policy": [_int],
    "locomp_amd_get_policy": [],
    "locomp_amd_release_workspaces": [_vp, _int],
    "locomp_amd_dequant_int4": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _int, _int, _vp],
    "locomp_amd_dequant_int8": [_vp, _vp, _vp, _i64, _i64, _i64, _i64, _int, _int, _vp],
    "locomp_amd_dequant_matvec_int4": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64, _i64,
                                       _int, _int, _int, _vp],
    "locomp_amd_dequant_matvec_int4_noalloc": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                               _i64, _int, _int, _int, _vp],
    "locomp_amd_dequant_matvec_int8": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                       _int, _int, _int, _vp],
    "locomp_amd_dequant_matvec_int4_silu_mul": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                                _i64, _int, _int, _int, _vp],
    "locomp_amd_launch": [ctypes.c_char_p, _int, _int, _int, _int, ctypes.POINTER(_vp),
                          ctypes.POINTER(_i64), _int, ctypes.POINTER(_int), _i64, _vp],
    "locomp_amd_quantize_int4": [_vp, _vp, _vp, _i64, _i64, _i64, _int, _int, _vp],
    "locomp_amd_quantize_int8": [_vp, _vp, _vp, _i64, _i64, _i64, _int, _vp],
    "locomp_amd_stream_read": [_vp, _i64, _vp, _vp],
    "locomp_amd_rms_norm": [_vp, _vp, _vp, _vp, _i64, _i64, ctypes.c_float, _int, _vp],
    "locomp_amd_dequant_matvec_int4_fused": [_vp, _vp, _vp, _vp, _i64, _i64, _i64, _i64, _i64,
                                             _i64, _int, _int, _int, _vp, ctypes.c_float, _vp,
                                             _int, _vp],
}

_lib = None


class LocompAMDError(RuntimeError):
    """A HIP error reported by the library (positive hipError_t)."""


def load(path: str | os.PathLike | None = None) -> ctypes.CDLL:
    """Load (once) and type the shared library; raises if it is not built."""
    global _lib
    if _lib is not None and path is None:
        return _lib
    p = Path(path) if path is not None else LIB_PATH
    if not p.exists():
        raise RuntimeError(
            f"locomp_amd HIP library not found at {p}; build it with "
            "`python -m locomp_amd.build` (there is no CPU fallback)")
    lib = ctypes.CDLL(str(p))
    for name, argtypes in SIGNATURES.items():
        fn = getattr(lib, name)
        fn.argtypes = argtypes
        fn.restype = ctypes.c_char_p if name == "locomp_amd_strerror" else ctypes.c_int
    v = lib.locomp_amd_abi_version()
    if v != ABI_VERSION:
        raise RuntimeError(f"locomp_amd ABI mismatch: library {v}, bindings {ABI_VERSION}")
    if path is None:
        _lib = lib
    return lib


def strerror(code: int) -> str:
    return load().locomp_amd_strerror(code).decode()


def check(code: int, what: str) -> None:
    """Map a library return code to a Python exception."""
    if code == OK:
        return
    if code < 0:
        raise ValueError(f"{what}: {strerror(code)} (code {code})")
    raise LocompAMDError(f"{what}: HIP error {code}: {strerror(code)}")


def set_policy(policy: int) -> None:
    check(load().locomp_amd_set_policy(policy), "set_policy")


def get_policy() -> int:
    return load().locomp_amd_get_policy()


def release_workspaces(stream=None, all_streams=True) -> None:
    """Free the library's cached fp32 workspaces (see the C entry)."""
    check(load().locomp_amd_release_workspaces(stream, 1 if all_streams else 0), "release_workspaces")
