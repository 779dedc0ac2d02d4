"""ctypes binding of the C ABI in include/bcjr_hip.h (libbcjr_hip.so).

This is the binding a maintainer would add on the reference side: it passes raw
device pointers, sizes and the current HIP stream.  torch supplies device memory
and streams only.  There is no fallback: if the library is missing or fails to
load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libbcjr_hip.so")

CODE_TABLE, CODE_1MAD, CODE_3INST, CODE_HYB = 0, 1, 2, 3
OP_FORWARD, OP_BACKWARD, OP_VITERBI = 0, 1, 2
BCJR_OK, BCJR_EINVAL, BCJR_EUNSUPPORTED, BCJR_EWORKSPACE, BCJR_EHIP = 0, -1, -2, -3, -4

# Every function include/bcjr_hip.h declares.
EXPORTS = (
    "bcjr_workspace_bytes", "bcjr_forward", "bcjr_forward_noalloc", "bcjr_forward_internals", "bcjr_forward_entropy", "bcjr_backward",
    "bcjr_viterbi", "bcjr_viterbi_constrained", "bcjr_viterbi_trace", "bcjr_decode", "bcjr_dequant", "bcjr_codebook", "bcjr_hadamard", "bcjr_rht", "bcjr_rht_batched",
    "bcjr_strerror", "bcjr_last_error", "bcjr_version",
)


class Problem(ctypes.Structure):
    """Mirror of bcjr_problem."""
    _fields_ = [
        ("L", ctypes.c_int), ("k", ctypes.c_int), ("V", ctypes.c_int),
        ("B", ctypes.c_int64), ("N", ctypes.c_int64),
        ("code", ctypes.c_int), ("Q", ctypes.c_int), ("t_per_seq", ctypes.c_int),
    ]


class BcjrError(RuntimeError):
    def __init__(self, status: int, what: str, detail: str):
        super().__init__(f"{what} failed: {detail or 'status %d' % status}")
        self.status = status


_lib = None


def load(path: str = LIB_PATH):
    """Load the shared library (after torch, so both use one HIP runtime)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(path):
        raise RuntimeError(
            f"BCJR HIP library not found at {path}; build it with "
            "`python -c 'import __graft_entry__ as g; g.build()'` (or make -C quant-2bit_amd/csrc)")
    import torch  # noqa: F401  (loads libamdhip64 so the library binds to the same runtime)
    lib = ctypes.CDLL(path)
    vp, sz, i32 = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    pp = ctypes.POINTER(Problem)
    lib.bcjr_workspace_bytes.argtypes = [pp, i32, ctypes.POINTER(sz)]
    lib.bcjr_forward.argtypes = [pp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.bcjr_forward_noalloc.argtypes = [pp, vp, vp, vp, vp, vp, vp]
    lib.bcjr_forward_internals.argtypes = [pp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.bcjr_forward_entropy.argtypes = [pp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.bcjr_backward.argtypes = [pp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.bcjr_viterbi.argtypes = [pp, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.bcjr_viterbi_constrained.argtypes = [pp, vp, vp, i32, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]
    lib.bcjr_decode.argtypes = [pp, vp, vp, vp, vp, vp, vp, vp]
    lib.bcjr_viterbi_trace.argtypes = [pp, vp, vp, vp, vp, vp]
    lib.bcjr_codebook.argtypes = [pp, vp, vp, vp]
    i64 = ctypes.c_int64
    lib.bcjr_hadamard.argtypes = [vp, vp, i64, i64, ctypes.c_float, vp]
    lib.bcjr_rht.argtypes = [vp, vp, i64, i64, vp, vp, i32, vp]
    lib.bcjr_rht_batched.argtypes = [vp, vp, i64, i64, i64, vp, vp, i32, vp]
    lib.bcjr_dequant.argtypes = [pp, vp, i32, vp, vp, i64, i64, i32, i32, ctypes.c_double, vp, vp]
    lib.bcjr_strerror.argtypes = [i32]
    for name in ("bcjr_workspace_bytes", "bcjr_forward", "bcjr_forward_noalloc", "bcjr_forward_internals", "bcjr_forward_entropy",
                 "bcjr_backward", "bcjr_viterbi", "bcjr_viterbi_constrained", "bcjr_viterbi_trace", "bcjr_decode", "bcjr_dequant", "bcjr_codebook", "bcjr_hadamard", "bcjr_rht", "bcjr_rht_batched"):
        getattr(lib, name).restype = i32
    for name in ("bcjr_strerror", "bcjr_last_error", "bcjr_version"):
        getattr(lib, name).restype = ctypes.c_char_p
    lib.bcjr_last_error.argtypes = []
    lib.bcjr_version.argtypes = []
    _lib = lib
    return lib


def check(status: int, what: str) -> None:
    if status != BCJR_OK:
        lib = load()
        detail = lib.bcjr_last_error().decode()
        raise BcjrError(status, what, f"{lib.bcjr_strerror(status).decode()}: {detail}")


def ptr(t) -> int | None:
    """Device pointer of a tensor (None for None)."""
    return None if t is None else t.data_ptr()
