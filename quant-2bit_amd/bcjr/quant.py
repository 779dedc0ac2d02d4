"""Chunked BCJR quantizer op around the node (src/bcjr/bcjr_quant.py:63-156).

Tiling follows src/qat/ste.py:138-159: an (m, n) matrix becomes
(n_col_blocks * n_row_blocks) sequences of Tx*Ty weights, block index
col_block * n_row_blocks + row_block, each 16x16 tile flattened row-major, then
viewed as (B, N, V) with N = Tx*Ty / V.  The RMS scale is detached
(bcjr_quant.py:140).  bcjr_quantize_weight wraps the rotated quantizer in the
random Hadamard transform (bcjr_quant.py:159-178) on the gfx950 FWHT kernels.
"""
from __future__ import annotations

import torch

from .forward_backward import K_BITS, L_BITS, V_DIM, bcjr_forward_backward
from .rht import apply_inverse_rht_gpu, apply_rht_gpu

TX = 16
TY = 16
BCJR_CHUNK = None  # whole batch per launch; workspace memory is bounded by the engine


def tile_for_viterbi(W, Tx=TX, Ty=TY):
    """(m, n) -> (n_col*n_row, Tx*Ty) sequences and (n_row, n_col)  (ste.py:138-149)."""
    m, n = W.shape
    if m % Tx or n % Ty:
        raise AssertionError(f"shape {(m, n)} not tileable by {(Tx, Ty)}")
    n_row, n_col = m // Tx, n // Ty
    seqs = W.reshape(m, n_col, Ty).permute(1, 0, 2).contiguous().reshape(n_col * n_row, Tx * Ty)
    return seqs, (n_row, n_col)


def untile_from_viterbi(recons, shape_info, shape_mn, Tx=TX, Ty=TY):
    """Inverse of tile_for_viterbi (ste.py:152-159)."""
    n_row, n_col = shape_info
    m, n = shape_mn
    return recons.reshape(n_col, m, Ty).permute(1, 0, 2).contiguous().reshape(m, n)


def _bcjr_chunk_forward(sequences_chunk, codebook, T_temp, preds=None, succs=None):
    """One node call returning soft (B, N, V) (bcjr_quant.py:63-82).  The
    reference dispatches on BCJR_MONOLITHIC / BCJR_FAST to one of its
    implementations; every one of them is this node here."""
    soft, _ = bcjr_forward_backward(sequences_chunk, codebook, T_temp, preds=preds, succs=succs)
    return soft


def graphed_bcjr_chunk_forward(sequences, codebook, T_temp, preds=None, succs=None):
    """Drop-in for src/bcjr/bcjr_graph.py:56-81 (BCJR_GRAPH): soft (B, N, V) from
    the node, which needs no graph capture to avoid per-step launches."""
    return _bcjr_chunk_forward(sequences, codebook, T_temp, preds, succs)


def reset_graph_cache():
    """src/bcjr/bcjr_graph.py:84-88.  No graphs are cached here."""


def bcjr_quantize_tiles(sequences, codebook, T_temp, preds=None, succs=None,
                        chunk_size=BCJR_CHUNK, use_checkpoint=True,
                        L=L_BITS, k=K_BITS, V=V_DIM):
    """(B, N, V) -> soft (B, N, V) (bcjr_quant.py:85-122).

    The reference splits B into chunks of chunk_size sequences and wraps each in
    an activation checkpoint to bound the memory of its (B, N, 2^L) lattices.
    Here one launch per direction covers the whole batch with memory bounded by
    the engine's workspace, and the node keeps only its inputs for the backward,
    so chunk_size and use_checkpoint are accepted for signature compatibility
    and not applied: the result is the same (sequences are independent) and a
    chunked loop would only multiply launches (a 237,568-tile layer at
    chunk_size=8 would be ~30,000 of them, each filling 8 of 256 CUs)."""
    soft, _ = bcjr_forward_backward(sequences, codebook, T_temp, L=L, k=k, V=V,
                                    preds=preds, succs=succs)
    return soft


def bcjr_quantize_weight_rotated(W_rotated, codebook, T_temp, preds=None, succs=None,
                                 chunk_size=BCJR_CHUNK, Tx=TX, Ty=TY,
                                 L=L_BITS, k=K_BITS, V=V_DIM):
    """Soft-quantize an already-rotated (m, n) weight (bcjr_quant.py:125-156)."""
    m, n = W_rotated.shape
    W_scale = W_rotated.detach().pow(2).mean().sqrt().clamp(min=1e-30)
    W_unit = W_rotated / W_scale
    seqs_flat, shape_info = tile_for_viterbi(W_unit, Tx, Ty)
    B, T_seq = seqs_flat.shape
    seqs = seqs_flat.view(B, T_seq // V, V)
    soft = bcjr_quantize_tiles(seqs, codebook, T_temp, preds, succs, chunk_size, L=L, k=k, V=V)
    W_q_unit = untile_from_viterbi(soft.contiguous().view(B, T_seq), shape_info, (m, n), Tx, Ty)
    return W_q_unit * W_scale


def bcjr_quantize_weight(W_latent, sign_l, sign_r, codebook, T_temp, preds=None, succs=None,
                         chunk_size=BCJR_CHUNK, Tx=TX, Ty=TY, L=L_BITS, k=K_BITS, V=V_DIM):
    """Soft-quantize W in its original basis: rotate, quantize, rotate back
    (bcjr_quant.py:159-178).  Gradients flow through both transforms and the
    BCJR node."""
    W_tilde = apply_rht_gpu(W_latent, sign_l, sign_r)
    W_tilde_q = bcjr_quantize_weight_rotated(W_tilde, codebook, T_temp, preds, succs, chunk_size=chunk_size,
                                             Tx=Tx, Ty=Ty, L=L, k=k, V=V)
    return apply_inverse_rht_gpu(W_tilde_q, sign_l, sign_r)


__all__ = ["TX", "TY", "tile_for_viterbi", "untile_from_viterbi", "bcjr_quantize_tiles",
           "bcjr_quantize_weight_rotated", "bcjr_quantize_weight", "graphed_bcjr_chunk_forward",
           "reset_graph_cache"]
