"""T -> 0 mode of the node: batched Viterbi encode, decode and 2-bit packing.

Drop-in for viterbi_encode_v_batched_cuda (src/viterbi/cuda_kernel.py:166-220),
generalised from its fixed L=16, k=2, V=2 to any supported (L, k, V), with the
tie rules and float32 rounding of the numpy encoder viterbi_encode_v
(src/viterbi/encode.py:250-307): lowest predecessor index and lowest final
state win ties; start_state = walk[0] >> kV.  Decoding replays
state_t = ((state_{t-1} << kV) | bits_t) & (2^L - 1) (encode.py:310-325,
src/qat/ste.py:270-283).
"""
from __future__ import annotations

import torch

from . import ops
from .forward_backward import _spec_for


def viterbi_encode_v_batched_hip(sequences, codebook, L=16, k=2, V=2, return_all=False):
    """sequences: (B, T) float32 with T = N*V; codebook (2^L, V).

    Returns (bitstreams (B, N) int32, start_states (B,) int32,
    recons (B, T) float32, mses (B,) float32); with return_all also the dict
    holding walk (B, N) and packed (B, ceil(N*kV/8)) uint8.
    """
    if not sequences.is_cuda:
        raise AssertionError("sequences must be a GPU tensor")
    if sequences.dtype != torch.float32 or codebook.dtype != torch.float32:
        raise AssertionError("sequences and codebook must be float32")
    if tuple(codebook.shape) != (1 << L, V):
        raise AssertionError(f"codebook must be ({1 << L}, {V}); got {tuple(codebook.shape)}")
    B, T = sequences.shape
    if T % V != 0:
        raise AssertionError(f"T={T} must be divisible by V={V}")
    spec, table = _spec_for(codebook, L, k, V)
    table = None if table is None else table.detach().contiguous()
    out = ops.viterbi(spec, sequences.reshape(B, T // V, V), table)
    res = (out["bitstream"], out["start"], out["recon"].reshape(B, T), out["mse"])
    if return_all:
        return res + (out,)
    return res


def viterbi_encode_v_batched_cuda(sequences, codebook):
    """The reference's entry point (src/viterbi/cuda_kernel.py:166-220), fixed at
    L=16, k=2, V=2: sequences (B, T) float32 GPU tensor with T even, codebook
    (65536, 2).  Returns (bitstreams (B, T/2) int32, start_states (B,) int32,
    recons (B, T) float32, mses (B,) float32)."""
    if not (sequences.is_cuda and codebook.is_cuda):
        raise AssertionError("sequences and codebook must be GPU tensors")
    if tuple(codebook.shape) != (65536, 2):
        raise AssertionError(f"codebook must be (65536, 2); got {tuple(codebook.shape)}")
    if sequences.dim() != 2 or sequences.shape[1] % 2:
        raise AssertionError(f"sequences must be (B, T) with T even; got {tuple(sequences.shape)}")
    return viterbi_encode_v_batched_hip(sequences, codebook, L=16, k=2, V=2)


def viterbi_encode_chunked(sequences, codebook, chunk=None, L=16, k=2, V=2):
    """Same contract as src/qat/ste.py:58-73.  The engine's memory use is bounded
    by its workspace, so the whole batch runs in one launch unless chunk is set."""
    if chunk is None or sequences.shape[0] <= chunk:
        return viterbi_encode_v_batched_hip(sequences, codebook, L, k, V)
    parts = [viterbi_encode_v_batched_hip(sequences[i:i + chunk], codebook, L, k, V)
             for i in range(0, sequences.shape[0], chunk)]
    return tuple(torch.cat([p[j] for p in parts], dim=0) for j in range(4))


def viterbi_decode_v_batched(bitstreams, start_states, codebook, L=16, k=2, V=2, packed=None, N=None):
    """Replay walks: returns (walks (B, N) int32, recons (B, N*V) float32)."""
    spec, table = _spec_for(codebook, L, k, V)
    table = None if table is None else table.detach().contiguous()
    walk, recon = ops.decode(spec, start_states, table, bitstream=bitstreams, packed=packed, N=N)
    return walk, recon.reshape(walk.shape[0], -1)


__all__ = ["viterbi_encode_v_batched_hip", "viterbi_encode_v_batched_cuda", "viterbi_encode_chunked",
           "viterbi_decode_v_batched"]
