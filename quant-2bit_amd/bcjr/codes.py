"""Trellis codebooks built on the GPU by the engine's generators, and the
resolution of any (2^L, V) codebook tensor to the source the kernels read.

Drop-in for the codebook producers the quantizer uses: decode_1mad_batch /
decode_3inst_batch materialised over all states (src/codes/ref.py:33-41, :76-91)
and make_hyb_codebook_gpu (src/qat/ste.py:376-392).  Values are bit-identical
to the reference generators.  The returned (2^L, V) float32 tensor also records
its generator, so bcjr_forward_backward / the Viterbi encoder hash c(s)
in-kernel instead of reading the table.

A table made elsewhere (the reference's own make_hyb_codebook_gpu, a copy made
by .to() or .clone(), a table loaded from disk) carries no record.
resolve_codebook recognises it by content: a (2^L, 1) table equal to the 1MAD or
3INST codebook, or a (2^L, 2) table equal to the HYB codebook of some LUT (the
LUT is read back out of the table), runs on the hashed / LUT kernels; anything
else runs on the table kernels, which read c(s) from the table.  Recognition
compares on the device and synchronises once per tensor (and again after an
in-place change of it); under stream capture an unrecognised table is not
examined and takes the table kernels.
"""
from __future__ import annotations

import warnings
import weakref

import numpy as np
import torch

from . import ops
from .ops import CODE_1MAD, CODE_3INST, CODE_HYB, CODE_TABLE, Spec


def _tag(cb: torch.Tensor, code: int, lut=None, Q: int = 9) -> torch.Tensor:
    cb._bcjr_code = code
    cb._bcjr_lut = lut
    cb._bcjr_Q = Q
    return cb


def make_1mad_codebook(L: int = 16, device="cuda") -> torch.Tensor:
    """(2^L, 1): ((byte sum of 34038481*s + 76625530) - 510) / 147.8, the table of
    src/codes/ref.py:33-41 (decode_1mad_batch), hashed on the device."""
    return _tag(ops.codebook(CODE_1MAD, L, device), CODE_1MAD)


def make_3inst_codebook(L: int = 16, device="cuda") -> torch.Tensor:
    """(2^L, 1): fp16-pair sum of (89226354*s + 64248484) & 0x8FFF8FFF ^ fp16(0.922), / 1.2447,
    the table of src/codes/ref.py:76-91 (decode_3inst_batch), hashed on the device."""
    return _tag(ops.codebook(CODE_3INST, L, device), CODE_3INST)


def make_hyb_codebook_gpu(lut_np, Q: int = 9, L_bits: int = 16, device="cuda") -> torch.Tensor:
    """(2^L, 2) from a (2^Q, 2) LUT: x = s*s + s, row (x >> (15-Q)) & (2^Q-1),
    second component negated when bit 15 of x is set (src/qat/ste.py:376-392)."""
    if torch.is_tensor(lut_np):
        lut = lut_np.detach().to(device=device, dtype=torch.float32).contiguous()
    else:
        lut = torch.from_numpy(np.ascontiguousarray(lut_np, dtype=np.float32)).to(device)
    if tuple(lut.shape) != (1 << Q, 2):
        raise AssertionError(f"LUT shape mismatch: {tuple(lut.shape)} != {(1 << Q, 2)}")
    return _tag(ops.codebook(CODE_HYB, L_bits, device, lut=lut, Q=Q), CODE_HYB, lut, Q)


def code_of(codebook: torch.Tensor) -> int:
    """Generator id recorded on a codebook (0 = plain table)."""
    return int(getattr(codebook, "_bcjr_code", 0))


# ---------------------------------------------------------------------------
# Resolution: (Spec, tensor the kernels read) for a codebook tensor.
# ---------------------------------------------------------------------------

# id(storage) -> (weakref to it, (offset, shape, stride, dtype), version, (code, Q, lut or None))
_SEEN: dict = {}
# Storages for which the capture warning of resolve_codebook was given.
_CAPTURE_WARNED = weakref.WeakSet()
# (device, code, L) -> generated codebook, for the comparisons
_GENERATED: dict = {}
# (L, Q) -> (rep_state (2^Q,) int64 or -1, negate (2^Q,) bool): for every LUT
# row one state that reads it, and whether that state reads its second
# component negated.
_HYB_READERS: dict = {}


def _generated(device: torch.device, code: int, L: int) -> torch.Tensor:
    key = (str(device), code, L)
    cb = _GENERATED.get(key)
    if cb is None:
        cb = ops.codebook(code, L, device)
        _GENERATED[key] = cb
    return cb


def _hyb_readers(L: int, Q: int):
    key = (L, Q)
    r = _HYB_READERS.get(key)
    if r is None:
        s = np.arange(1 << L, dtype=np.uint64)
        x = (s * s + s) & np.uint64(0xFFFFFFFF)
        idx = ((x >> np.uint64(15 - Q)) & np.uint64((1 << Q) - 1)).astype(np.int64)
        neg = ((x >> np.uint64(15)) & np.uint64(1)).astype(bool)
        rep = np.full(1 << Q, -1, dtype=np.int64)
        rep_neg = np.zeros(1 << Q, dtype=bool)
        # prefer a state that reads the row unnegated; the last write wins, so
        # write the negated readers first
        for want in (True, False):
            sel = np.nonzero(neg == want)[0]
            rep[idx[sel]] = sel
            rep_neg[idx[sel]] = want
        r = (rep, rep_neg)
        _HYB_READERS[key] = r
    return r


def _recognise(cb: torch.Tensor, L: int, V: int):
    """(code, Q, lut) for a float32 contiguous device table, by content."""
    dev = cb.device
    if V == 1:
        for code in (CODE_3INST, CODE_1MAD):
            if torch.equal(cb, _generated(dev, code, L)):
                return code, 0, None
        return CODE_TABLE, 0, None
    if V == 2 and L <= 16:
        for Q in (9,) + tuple(q for q in range(1, 13) if q != 9):
            rep, rep_neg = _hyb_readers(L, Q)
            rep_t = torch.from_numpy(np.maximum(rep, 0)).to(dev)
            lut = cb.index_select(0, rep_t).clone()
            sign = torch.from_numpy(np.where(rep_neg, -1.0, 1.0).astype(np.float32)).to(dev)
            lut[:, 1] *= sign
            lut[torch.from_numpy(rep < 0).to(dev)] = 0.0
            lut = lut.contiguous()
            if torch.equal(cb, ops.codebook(CODE_HYB, L, dev, lut=lut, Q=Q)):
                return CODE_HYB, Q, lut
    return CODE_TABLE, 0, None


# Bits per step (k*V) for which the generator codes (1MAD, 3INST, HYB) have
# kernels of their own; at k*V = 1 only the table kernels are built.
GENERATOR_KV = (2, 4)


def _canonical(device) -> torch.device:
    """torch.device with the index filled in ('cuda' -> 'cuda:<current>')."""
    device = torch.device(device)
    if device.type == "cuda" and device.index is None:
        return torch.device("cuda", torch.cuda.current_device())
    return device


def resolve_codebook(codebook: torch.Tensor, L: int, k: int, V: int, device: torch.device):
    """(Spec, table) for a (2^L, V) codebook used on `device`: table is the
    float32 device tensor the kernels read (the codebook itself for table
    kernels, the (2^Q, 2) LUT for HYB) or None for hashed codes.

    Raises AssertionError when the codebook's shape is not (2^L, V) or it lives
    on another device than the sequences (the reference fails there too: a
    device mismatch in its einsum, src/bcjr/forward_backward.py:100).

    The recognition of an untagged table is cached per storage and re-run when
    the tensor's version counter moves (any in-place torch op on it).  Writes
    that bypass the counter -- through `.data`, or by another kernel or library
    writing through `data_ptr()` -- leave the cached result in place, and a
    table recognised as 1MAD/3INST/HYB would keep running on the hashed / LUT
    kernels with its old contents.  Call forget(codebook) after such a write
    (the reference reads the table on every call and has no such cache)."""
    if tuple(codebook.shape) != (1 << L, V):
        raise AssertionError(f"codebook must be ({1 << L}, {V}); got {tuple(codebook.shape)}")
    device = _canonical(device)
    if _canonical(codebook.device) != device:
        raise AssertionError(f"codebook is on {codebook.device} but the sequences are on {device}")
    if k * V not in GENERATOR_KV:
        # No hashed or LUT kernels at this shape: any codebook is a table.
        table = codebook.detach()
        if table.dtype != torch.float32 or not table.is_contiguous():
            table = table.to(torch.float32).contiguous()
        return Spec(L, k, V, CODE_TABLE), table
    code = getattr(codebook, "_bcjr_code", None)
    if code is not None:
        if code == CODE_HYB:
            lut = codebook._bcjr_lut
            if _canonical(lut.device) != device:
                raise AssertionError(f"HYB LUT is on {lut.device} but the sequences are on {device}")
            return Spec(L, k, V, CODE_HYB, int(codebook._bcjr_Q)), lut
        if code != CODE_TABLE:
            return Spec(L, k, V, int(code)), None
    table = codebook.detach()
    if table.dtype != torch.float32 or not table.is_contiguous():
        table = table.to(torch.float32).contiguous()
    # Keyed by the storage (views and new tensor objects over it share the
    # entry); the weak reference makes a freed storage's entry unreachable, so
    # a new allocation at the same address is examined afresh.
    storage = codebook.untyped_storage()
    view = (codebook.storage_offset(), tuple(codebook.shape), tuple(codebook.stride()), codebook.dtype)
    hit = _SEEN.get(id(storage))
    res = None
    if hit is not None:
        ref, hview, version, r = hit
        if ref() is storage and hview == view and version == codebook._version:
            res = r
    if res is None:
        if torch.cuda.is_current_stream_capturing():
            # Recognition compares on the device and reads the verdict back, which
            # a capture cannot do: the table runs on the table kernels (correct,
            # but several times slower than the generator kernels at L = 16).
            if storage not in _CAPTURE_WARNED:
                _CAPTURE_WARNED.add(storage)
                warnings.warn(
                    "bcjr: a codebook table first seen inside a graph capture runs on the table kernels; "
                    "call the node (or bcjr.codes.resolve_codebook) on it once before capturing so that a "
                    "1MAD/3INST/HYB table reaches its generator kernels", RuntimeWarning, stacklevel=3)
            return Spec(L, k, V, CODE_TABLE), table
        res = _recognise(table, L, V)
        for dead in [k_ for k_, v in _SEEN.items() if v[0]() is None]:
            del _SEEN[dead]
        _SEEN[id(storage)] = (weakref.ref(storage), view, codebook._version, res)
    code, Q, lut = res
    if code == CODE_TABLE:
        return Spec(L, k, V, CODE_TABLE), table
    if code == CODE_HYB:
        return Spec(L, k, V, CODE_HYB, Q), lut
    return Spec(L, k, V, code), None


def forget(codebook: torch.Tensor) -> None:
    """Drop the recognition result cached for codebook's storage, so the next
    resolve_codebook examines its contents afresh.  Needed only after a write
    that bypasses the tensor's version counter (see resolve_codebook); a
    generator tag (make_*_codebook) is not affected."""
    _SEEN.pop(id(codebook.untyped_storage()), None)


__all__ = ["make_1mad_codebook", "make_3inst_codebook", "make_hyb_codebook_gpu", "code_of", "resolve_codebook",
           "forget"]
