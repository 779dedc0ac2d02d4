"""The numpy-facing Viterbi API of src/viterbi/encode.py on the gfx950 kernels.

Same names, arguments and return values as the reference module: a sequence
is a numpy array (encoded in float32), ``decode_fn`` maps a uint32 array of states to their
codewords ((n,) for V = 1, (n, V) otherwise), and results come back as numpy
values.  The codebook is materialised once per call (precompute_codebook_v,
encode.py:233-247) and every encode is one launch of the min-sum kernel (two
for tail-biting), so the results are those of the direct form of
viterbi_encode_v (encode.py:250-307): the float32 rounding of
(c - w)^2 summed over v, then added to the best predecessor cost; the lowest
predecessor index and the lowest final state win ties.  mse is
float(np.mean((recon - sequence) ** 2)), computed here exactly as the
reference computes it.

viterbi_encode_v_batched (encode.py:425-495) returns the same values as
viterbi_encode_v on each sequence, which is what the reference's own gate asks
of it (src/tripwires/test_viterbi_batched.py:27-72).  return_trace=True adds
the (T/V, 2^L) lattices of cumulative costs and chosen predecessor states, from
one more launch (bcjr_viterbi_trace) with the same rounding and tie rules.
"""
from __future__ import annotations

import hashlib
from collections import OrderedDict

import numpy as np
import torch

from . import ops
from .viterbi import (viterbi_decode_v_batched, viterbi_encode_constrained_v_batched_hip,
                      viterbi_encode_tailbiting_v_batched_hip, viterbi_encode_v_batched_hip)


def precompute_predecessors_v(L, k, V):
    """(2^L, 2^(kV)) int32: preds[s, p] = (p << (L - kV)) | (s >> kV) (encode.py:218-230)."""
    kV = k * V
    s = np.arange(1 << L, dtype=np.int64)
    p = np.arange(1 << kV, dtype=np.int64)
    return ((p[None, :] << (L - kV)) | (s[:, None] >> kV)).astype(np.int32)


def precompute_predecessors(L, k):
    """V = 1 form (encode.py:22-37)."""
    return precompute_predecessors_v(L, k, 1)


def precompute_codebook_v(L, V, decode_fn):
    """decode_fn over every state as a (2^L, V) float32 array (encode.py:233-247)."""
    n = 1 << L
    result = np.asarray(decode_fn(np.arange(n, dtype=np.uint32)))
    if result.ndim == 1:
        result = result[:, None]
    if result.shape != (n, V):
        raise AssertionError(f"decode_fn returned shape {result.shape}, expected ({n}, {V})")
    return result.astype(np.float32)


def precompute_codebook(L, decode_fn):
    """decode_fn over every state, float32 (encode.py:40-44)."""
    n = 1 << L
    return np.asarray(decode_fn(np.arange(n, dtype=np.uint32))).astype(np.float32)


def _device():
    if not torch.cuda.is_available():
        raise RuntimeError("the Viterbi engine runs on the GPU; no HIP device is visible")
    return torch.device("cuda", torch.cuda.current_device())


# Device codebooks of the numpy-facing calls, keyed by their contents: each call
# evaluates decode_fn (as the reference does, encode.py:233-247) and reuses the
# device tensor of an identical table, so its recognition (resolve_codebook) is
# cached across calls instead of re-run on a new tensor every time.  Keyed by
# content, not by decode_fn, a decode_fn whose table changes (a LUT updated in
# place) gets a fresh tensor.  A few tables at most are kept.
_GPU_TABLES: "OrderedDict[tuple, torch.Tensor]" = OrderedDict()
_GPU_TABLES_MAX = 8


def _gpu_codebook(L, V, decode_fn):
    table = precompute_codebook_v(L, V, decode_fn)
    dev = _device()
    key = (L, V, str(dev), hashlib.blake2b(table.tobytes(), digest_size=16).digest())
    cb = _GPU_TABLES.get(key)
    if cb is None:
        cb = torch.from_numpy(table).to(dev)
        _GPU_TABLES[key] = cb
        while len(_GPU_TABLES) > _GPU_TABLES_MAX:
            _GPU_TABLES.popitem(last=False)
    else:
        _GPU_TABLES.move_to_end(key)
    return cb


def _sequences(sequences, V):
    x = np.asarray(sequences, dtype=np.float32)
    if x.shape[-1] % V:
        raise AssertionError(f"Sequence length {x.shape[-1]} must be divisible by V={V}")
    return x


def _mse(recon, sequence):
    return float(np.mean((recon - sequence) ** 2))


def viterbi_encode_v(sequence, L, k, V, decode_fn, return_trace=False):
    """(bitstream (T/V,) int32, start_state int, recon (T,) float32, mse float)
    (encode.py:250-307); with return_trace=True also trace_err (T/V, 2^L)
    float32, the cumulative cost of every state after every step, and
    backpointers (T/V, 2^L) int32, the predecessor each state's minimum chose."""
    x = _sequences(sequence, V)
    cb = _gpu_codebook(L, V, decode_fn)
    xs = torch.from_numpy(x[None]).to(cb.device)
    bits, start, recon, _ = viterbi_encode_v_batched_hip(xs, cb, L=L, k=k, V=V)
    recon = recon[0].cpu().numpy()
    out = (bits[0].cpu().numpy(), int(start[0]), recon, _mse(recon, np.asarray(sequence)))
    if not return_trace:
        return out
    trace, backptr = ops.viterbi_trace(ops.Spec(L, k, V, ops.CODE_TABLE), xs.reshape(1, -1, V), cb)
    return out + (trace[0].cpu().numpy(), backptr[0].cpu().numpy())


def viterbi_encode(sequence, L, k, decode_fn, return_trace=False):
    """V = 1 form (encode.py:47-87)."""
    return viterbi_encode_v(sequence, L, k, 1, decode_fn, return_trace)


def viterbi_decode_v(bitstream, start_state, L, k, V, decode_fn):
    """Replay the walk and return its codewords, (T,) float32 (encode.py:310-325)."""
    cb = _gpu_codebook(L, V, decode_fn)
    bits = torch.as_tensor(np.asarray(bitstream, dtype=np.int32)[None], device=cb.device)
    start = torch.tensor([int(start_state)], dtype=torch.int32, device=cb.device)
    _, recon = viterbi_decode_v_batched(bits, start, cb, L=L, k=k, V=V)
    return recon[0].cpu().numpy()


def viterbi_decode(bitstream, start_state, L, k, decode_fn):
    """V = 1 form (encode.py:90-102)."""
    return viterbi_decode_v(bitstream, start_state, L, k, 1, decode_fn)


def viterbi_encode_v_batched(sequences, L, k, V, decode_fn):
    """(bitstreams (B, T/V) int32, start_states (B,) int32, recons (B, T) float32,
    mses (B,) float32) (encode.py:425-495)."""
    x = _sequences(sequences, V)
    cb = _gpu_codebook(L, V, decode_fn)
    bits, start, recon, _ = viterbi_encode_v_batched_hip(torch.from_numpy(x).to(cb.device), cb, L=L, k=k, V=V)
    recon = recon.cpu().numpy()
    mses = ((recon - np.asarray(sequences).astype(np.float32)) ** 2).mean(axis=1).astype(np.float32)
    return bits.cpu().numpy(), start.cpu().numpy().astype(np.int32), recon, mses


def viterbi_encode_constrained_v(sequence, L, k, V, decode_fn, overlap_bits, overlap_value):
    """Encode with the first state's top overlap_bits bits and the last state's
    bottom overlap_bits bits equal to overlap_value (encode.py:328-389); raises
    RuntimeError when no walk meets it.  overlap_bits <= L - k*V."""
    x = _sequences(sequence, V)
    cb = _gpu_codebook(L, V, decode_fn)
    bits, start, recon, _ = viterbi_encode_constrained_v_batched_hip(
        torch.from_numpy(x[None]).to(cb.device), cb, [int(overlap_value)], overlap_bits, L=L, k=k, V=V)
    start = int(start[0])
    if start < 0:
        raise RuntimeError(f"No valid tail-biting walk for overlap_value={overlap_value}")
    recon = recon[0].cpu().numpy()
    return bits[0].cpu().numpy(), start, recon, _mse(recon, np.asarray(sequence))


def viterbi_encode_constrained(sequence, L, k, decode_fn, overlap_bits, overlap_value):
    """V = 1 form (encode.py:105-172)."""
    return viterbi_encode_constrained_v(sequence, L, k, 1, decode_fn, overlap_bits, overlap_value)


def viterbi_encode_tailbiting_v(sequence, L, k, V, decode_fn):
    """Tail-biting encode, Algorithm 4 (encode.py:392-422): (bitstream, start_state,
    recon, mse, overlap_value)."""
    x = _sequences(sequence, V)
    cb = _gpu_codebook(L, V, decode_fn)
    bits, start, recon, _, ov = viterbi_encode_tailbiting_v_batched_hip(
        torch.from_numpy(x[None]).to(cb.device), cb, L=L, k=k, V=V)
    start, ov = int(start[0]), int(ov[0])
    if start < 0:
        raise RuntimeError(f"No valid tail-biting walk for overlap_value={ov}")
    recon = recon[0].cpu().numpy()
    return bits[0].cpu().numpy(), start, recon, _mse(recon, np.asarray(sequence)), ov


def viterbi_encode_tailbiting(sequence, L, k, decode_fn):
    """V = 1 form (encode.py:175-216)."""
    return viterbi_encode_tailbiting_v(sequence, L, k, 1, decode_fn)


__all__ = ["precompute_predecessors", "precompute_predecessors_v", "precompute_codebook",
           "precompute_codebook_v", "viterbi_encode", "viterbi_encode_v", "viterbi_decode", "viterbi_decode_v",
           "viterbi_encode_v_batched", "viterbi_encode_constrained", "viterbi_encode_constrained_v",
           "viterbi_encode_tailbiting", "viterbi_encode_tailbiting_v"]
