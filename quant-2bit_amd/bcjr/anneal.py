"""Temperature source and diagnostics around the BCJR node (src/bcjr/anneal.py).

cosine_temperature_schedule is the T source of the annealed QAT loop
(anneal.py:53-61); measure_ptq_residual gives its natural starting point
T_0 (anneal.py:110-140, implemented in .ste).  entropy_diagnostic
(anneal.py:143-184) reports the mean marginal entropy of a layer's tiles: the
reference materialises P (B', N, 2^L) through return_internals=True on at most
32 sampled tiles per weight and reduces -(P log P); here the entropy is a
fused output of the forward kernel (bcjr_forward_entropy), so no (B, N, 2^L)
tensor exists and every tile can be included (max_tiles=None).
"""
from __future__ import annotations

import math

import torch

from . import ops
from .codes import resolve_codebook
from .forward_backward import K_BITS, L_BITS, V_DIM, _check_args
from .quant import TX, TY, tile_for_viterbi
from .rht import apply_rht_gpu
from .ste import _f32_cuda, _quantized_linears, _rms, measure_ptq_residual


def cosine_temperature_schedule(step, total_steps, T_0, T_min):
    """Cosine decay from T_0 at step 0 to T_min at step total_steps - 1, and T_min
    from then on (anneal.py:53-61)."""
    if total_steps <= 1:
        return T_min
    frac = min(max(step, 0), total_steps - 1) / (total_steps - 1)
    return T_min + 0.5 * (T_0 - T_min) * (1.0 + math.cos(math.pi * frac))


def bcjr_marginal_entropy(sequences, codebook, T_temp, L=L_BITS, k=K_BITS, V=V_DIM):
    """Marginal entropy H[b, t] = -sum_s P_t(s) ln P_t(s) in nats, (B, N) float32: what
    src/bcjr/anneal.py:143-184 (entropy_diagnostic) reduces from the (B, N, 2^L)
    marginals of return_internals=True, here fused into the forward.

    Same arguments as bcjr_forward_backward (T_temp may be per sequence); no
    gradient.  Bounds: 0 <= H <= L ln 2, the upper one reached by the uniform
    marginals of T -> inf."""
    _check_args(sequences, codebook, L, k, V, None, None)
    spec, table = resolve_codebook(codebook, L, k, V, sequences.device)
    _, _, H = ops.forward_entropy(spec, sequences, T_temp, table)
    return H


def entropy_diagnostic(qat_layer, max_tiles=32, Tx=TX, Ty=TY, k=K_BITS, generator=None):
    """Average marginal entropy (nats) over the tiles of every quantized linear of
    a layer that is in BCJR mode (anneal.py:143-184).

    A quantized linear is any object with W_latent, sign_l, sign_r, codebook_gpu
    and T_temp (the layer itself, its modules, or an iterable of them); one with
    a quant_mode other than "bcjr" is skipped, as in the reference.  Each weight
    is rotated, RMS-normalised and tiled as the quantizer sees it; at most
    max_tiles tiles per weight are drawn with torch.randperm (pass a generator
    for a fixed draw), or all of them with max_tiles=None.  Returns nan when no
    tile was seen."""
    total_h, total_n = 0.0, 0
    with torch.no_grad():
        for ql in _quantized_linears(qat_layer):
            if getattr(ql, "quant_mode", "bcjr") != "bcjr":
                continue
            cb = ql.codebook_gpu
            L = int(cb.shape[0]).bit_length() - 1
            V = int(cb.shape[1])
            dev = ql.W_latent.device
            W_tilde = apply_rht_gpu(ql.W_latent.float(), _f32_cuda(ql.sign_l, dev), _f32_cuda(ql.sign_r, dev))
            seqs_flat, _ = tile_for_viterbi(W_tilde / _rms(W_tilde), Tx, Ty)
            B, n_w = seqs_flat.shape
            seqs = seqs_flat.view(B, n_w // V, V)
            if max_tiles is not None and B > max_tiles:
                idx = torch.randperm(B, device=seqs.device, generator=generator)[:max_tiles]
                seqs = seqs[idx]
            H = bcjr_marginal_entropy(seqs, cb, ql.T_temp, L=L, k=k, V=V)
            total_h += float(H.double().sum())
            total_n += H.numel()
    if total_n == 0:
        return float("nan")
    return total_h / total_n


__all__ = ["cosine_temperature_schedule", "bcjr_marginal_entropy", "entropy_diagnostic", "measure_ptq_residual"]
