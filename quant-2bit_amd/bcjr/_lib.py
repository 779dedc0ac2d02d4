"""Loaders of the engine's two libraries.

libbcjr_torch.so registers the `bcjr` torch operators in C++ (TORCH_LIBRARY,
csrc/bcjr_torch.cpp) over the C ABI of libbcjr_hip.so; the package calls the
engine only through those operators (torch.ops.bcjr.*).  load() is the ctypes
binding of the raw C ABI in include/bcjr_hip.h -- the binding a maintainer
would add on a reference side without torch: raw device pointers, sizes and a
HIP stream -- used by the ABI tests.  There is no fallback: if a library is
missing or fails to load, every entry point raises.
"""
from __future__ import annotations

import ctypes
import os
import re

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libbcjr_hip.so")
OPS_PATH = os.path.join(_HERE, "libbcjr_torch.so")

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


_ops_loaded = False


def load_ops():
    """torch.ops.bcjr, after loading libbcjr_torch.so (once).  It links
    libbcjr_hip.so from its own directory."""
    global _ops_loaded
    import torch
    if not _ops_loaded:
        if not os.path.exists(OPS_PATH):
            raise RuntimeError(
                f"BCJR torch operator library not found at {OPS_PATH}; build it with "
                "`python -c 'import __graft_entry__ as g; g.build()'` (or make -C quant-2bit_amd/csrc)")
        torch.ops.load_library(OPS_PATH)
        _ops_loaded = True
    return torch.ops.bcjr


# A failed C ABI call inside an operator raises RuntimeError("bcjr status <n>:
# <entry point> failed: <detail>"); run_op re-raises it as BcjrError.
_STATUS = re.compile(r"bcjr status (-?\d+): (\w+) failed: ([^\n]*)")


def run_op(op, *args):
    """op(*args), with a failed C ABI call re-raised as BcjrError (under
    torch.compile the operator is traced as it is)."""
    import torch
    if torch.compiler.is_compiling():
        return op(*args)
    try:
        return op(*args)
    except RuntimeError as e:
        m = _STATUS.search(str(e))
        if m is None:
            raise
        raise BcjrError(int(m.group(1)), m.group(2), m.group(3)) from None


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
