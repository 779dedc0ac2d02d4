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
from .codes import resolve_codebook


def viterbi_encode_v_batched_hip(sequences, codebook, L=16, k=2, V=2, return_all=False):
    """Batched Viterbi (src/viterbi/cuda_kernel.py:166-220 viterbi_encode_v_batched_cuda,
    src/viterbi/encode.py:425-495 viterbi_encode_v_batched) for any L, k, V.

    sequences: (B, T) float32 with T = N*V; codebook (2^L, V).

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
    spec, table = resolve_codebook(codebook, L, k, V, sequences.device)
    out = ops.viterbi(spec, sequences.reshape(B, T // V, V), table)
    res = (out["bitstream"], out["start"], out["recon"].reshape(B, T), out["mse"])
    if return_all:
        return res + (out,)
    return res


def _check_batch(sequences, codebook, L, V):
    if not sequences.is_cuda:
        raise AssertionError("sequences must be a GPU tensor")
    if sequences.dtype != torch.float32 or codebook.dtype != torch.float32:
        raise AssertionError("sequences and codebook must be float32")
    if tuple(codebook.shape) != (1 << L, V):
        raise AssertionError(f"codebook must be ({1 << L}, {V}); got {tuple(codebook.shape)}")
    if sequences.dim() != 2 or sequences.shape[1] % V:
        raise AssertionError(f"sequences must be (B, T) with T divisible by V={V}; got {tuple(sequences.shape)}")


def viterbi_encode_constrained_v_batched_hip(sequences, codebook, overlap_values, overlap_bits=None,
                                             L=16, k=2, V=2, return_all=False):
    """Batched viterbi_encode_constrained_v (src/viterbi/encode.py:328-389): the
    walk of sequence b starts in a state whose top overlap_bits bits equal
    overlap_values[b] and ends in one whose bottom overlap_bits bits do
    (overlap_bits defaults to L - k*V, the tail-biting overlap; at most that).

    Returns (bitstreams, start_states, recons, mses) as viterbi_encode_v_batched_hip;
    start_states[b] is -1 where no walk meets the constraint (the reference
    raises RuntimeError there)."""
    _check_batch(sequences, codebook, L, V)
    kV = k * V
    ob = L - kV if overlap_bits is None else int(overlap_bits)
    B, T = sequences.shape
    spec, table = resolve_codebook(codebook, L, k, V, sequences.device)
    ov = torch.as_tensor(overlap_values, dtype=torch.int64, device=sequences.device).reshape(-1)
    if ov.numel() == 1:
        ov = ov.expand(B)
    out = ops.viterbi(spec, sequences.reshape(B, T // V, V), table, overlap=ov.to(torch.int32),
                      overlap_bits=ob)
    res = (out["bitstream"], out["start"], out["recon"].reshape(B, T), out["mse"])
    return res + (out,) if return_all else res


def viterbi_encode_tailbiting_v_batched_hip(sequences, codebook, L=16, k=2, V=2, return_all=False):
    """Batched viterbi_encode_tailbiting_v (Algorithm 4, src/viterbi/encode.py:392-422;
    V = 1: :175-216) in two Viterbi launches: every sequence rotated right by
    N//2 steps and encoded, the top L - k*V bits of each rotated walk's state at
    step N//2 taken as its overlap, the originals encoded under that
    constraint.  Returns (bitstreams, start_states, recons, mses, overlaps (B,)
    int32)."""
    _check_batch(sequences, codebook, L, V)
    kV = k * V
    B, T = sequences.shape
    N = T // V
    spec, table = resolve_codebook(codebook, L, k, V, sequences.device)
    steps = sequences.reshape(B, N, V)
    rot = ops.viterbi(spec, torch.roll(steps, N // 2, dims=1).contiguous(), table, want_packed=False)
    overlap = (rot["walk"][:, N // 2] >> kV).to(torch.int32)
    out = ops.viterbi(spec, steps, table, overlap=overlap, overlap_bits=L - kV)
    res = (out["bitstream"], out["start"], out["recon"].reshape(B, T), out["mse"], overlap)
    return res + (out,) if return_all else res


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
    """Replay walks (src/viterbi/encode.py:310-325 viterbi_decode_v, batched as
    src/qat/ste.py:270-283 _replay_walks): returns (walks (B, N) int32, recons
    (B, N*V) float32)."""
    spec, table = resolve_codebook(codebook, L, k, V, start_states.device)
    walk, recon = ops.decode(spec, start_states, table, bitstream=bitstreams, packed=packed, N=N)
    return walk, recon.reshape(walk.shape[0], -1)


__all__ = ["viterbi_encode_v_batched_hip", "viterbi_encode_v_batched_cuda", "viterbi_encode_chunked",
           "viterbi_decode_v_batched", "viterbi_encode_constrained_v_batched_hip",
           "viterbi_encode_tailbiting_v_batched_hip"]
