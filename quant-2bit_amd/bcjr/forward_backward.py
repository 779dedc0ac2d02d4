"""BCJR forward-backward node on the bitshift trellis, backed by gfx950 HIP kernels.

Drop-in for src/bcjr/forward_backward.py (bcjr_forward_backward,
build_pred_succ_tables, L_BITS/K_BITS/V_DIM) and src/bcjr/bcjr_monolithic.py
(bcjr_forward_backward_monolithic): same call signatures, tensor layouts,
return values and assertion behaviour.  The whole forward (alpha and beta
recursions, marginals, soft codeword, log Z) is one kernel launch, and the
backward is one more; autograd saves only the inputs.

Trellis (forward_backward.py:1-45): S = 2^L states, kV = k*V bits per step,
next = ((s << kV) | c) & (S-1); emission ll_t(s) = -||c(s) - w_t||^2 / T;
log_alpha_{-1} = 0 (free start), log_beta_{N-1} = 0 (free end).

Codebooks.  `codebook` is the (2^L, V) float32 table, as in the reference.  A
table made by bcjr.codes (make_1mad_codebook, make_3inst_codebook,
make_hyb_codebook_gpu) carries its generator, and the kernels then hash c(s)
in-kernel instead of reading the table; the values are bit-identical.
"""
from __future__ import annotations

import torch

from . import ops
from .ops import CODE_HYB, CODE_TABLE, Spec

L_BITS = 16
K_BITS = 2
V_DIM = 2


def build_pred_succ_tables(L=L_BITS, k=K_BITS, V=V_DIM, device="cuda"):
    """(preds, succs) int64 (S, 2^kV): preds[s,p] = (p << (L-kV)) | (s >> kV),
    succs[s,c] = ((s << kV) | c) & (S-1)  (forward_backward.py:62-86).

    The kernels never read these tables (the structure is implicit); they are
    built for callers that pass or cache them."""
    S = 1 << L
    kV = k * V
    s_arr = torch.arange(S, dtype=torch.int64, device=device)
    c_arr = torch.arange(1 << kV, dtype=torch.int64, device=device)
    preds = (c_arr.unsqueeze(0) << (L - kV)) | (s_arr >> kV).unsqueeze(1)
    succs = ((s_arr.unsqueeze(1) << kV) & (S - 1)) | c_arr.unsqueeze(0)
    return preds, succs


def _spec_for(codebook, L, k, V):
    """Spec and the pointer source for the kernels (table, HYB LUT or None)."""
    code = getattr(codebook, "_bcjr_code", CODE_TABLE)
    if code == CODE_TABLE:
        return Spec(L, k, V, CODE_TABLE), codebook
    if code == CODE_HYB:
        return Spec(L, k, V, CODE_HYB, int(codebook._bcjr_Q)), codebook._bcjr_lut
    return Spec(L, k, V, int(code)), None


def _check_args(sequences, codebook, L, k, V, preds, succs):
    # Same conditions as forward_backward.py:206-207, plus table shapes.
    if not (sequences.dim() == 3 and sequences.shape[-1] == V):
        raise AssertionError(f"sequences must be (B, N, V={V}); got {tuple(sequences.shape)}")
    if tuple(codebook.shape) != (1 << L, V):
        raise AssertionError(f"codebook must be ({1 << L}, {V}); got {tuple(codebook.shape)}")
    for name, tab in (("preds", preds), ("succs", succs)):
        if tab is not None and tuple(tab.shape) != (1 << L, 1 << (k * V)):
            raise AssertionError(f"{name} must be ({1 << L}, {1 << (k * V)}); got {tuple(tab.shape)}")
    if not sequences.is_cuda:
        raise AssertionError("bcjr_forward_backward runs on the GPU; sequences are on "
                             f"{sequences.device}")


class BcjrFunction(torch.autograd.Function):
    """One autograd node: forward = bcjr_forward, backward = bcjr_backward.

    Saves only (sequences, T, table); the backward recomputes the recursions
    on the GPU (the O(B*N*S) lattice never exists in memory)."""

    @staticmethod
    def forward(ctx, sequences, T, table, spec):
        soft, logZ = ops.forward(spec, sequences, T, table)
        ctx.spec = spec
        ctx.in_dtype = sequences.dtype
        ctx.save_for_backward(sequences, T if torch.is_tensor(T) else None,
                              table if table is not None else None)
        ctx.T_value = None if torch.is_tensor(T) else float(T)
        return soft.to(sequences.dtype), logZ.to(sequences.dtype)

    @staticmethod
    def backward(ctx, g_soft, g_logZ):
        sequences, T_saved, table = ctx.saved_tensors
        T = T_saved if T_saved is not None else ctx.T_value
        if g_soft is None and g_logZ is None:
            return None, None, None, None
        d = ops.backward(ctx.spec, sequences, T, table, g_soft, g_logZ)
        return d.to(ctx.in_dtype), None, None, None


def bcjr_forward_backward(sequences, codebook, T_temp,
                          L=L_BITS, k=K_BITS, V=V_DIM,
                          preds=None, succs=None, return_internals=False):
    """Full BCJR forward-backward (forward_backward.py:190-232).

    sequences: (B, N, V) float, requires_grad allowed.
    codebook:  (2^L, V) float32 (no gradient).
    T_temp:    temperature > 0: python float, 0-d tensor, or (B,) tensor (one
               per sequence, for batching several tensors in one call).

    Returns (soft (B,N,V), log_Z (B,)), or with return_internals
    (soft, log_Z, P, log_alpha, log_beta) with the last three (B, N, 2^L).
    Both soft and log_Z are differentiable with respect to sequences.
    """
    _check_args(sequences, codebook, L, k, V, preds, succs)
    spec, table = _spec_for(codebook, L, k, V)
    if return_internals:
        soft, logZ, P, la, lb = ops.forward_internals(spec, sequences, T_temp, _as_table(spec, table))
        dt = sequences.dtype
        return soft.to(dt), logZ.to(dt), P, la, lb
    return BcjrFunction.apply(sequences, T_temp, _as_table(spec, table), spec)


def _as_table(spec, table):
    if table is None:
        return None
    return table.detach().to(torch.float32).contiguous()


def bcjr_forward_backward_monolithic(sequences, codebook, T_temp,
                                     L=L_BITS, k=K_BITS, V=V_DIM,
                                     preds=None, succs=None,
                                     return_internals=False):
    """Drop-in for bcjr_monolithic.py:246-262: one autograd node, returns (soft, None).

    The reference variant is fixed to its module defaults (L=16, kV=4); this
    one honours L, k and V."""
    soft, _ = bcjr_forward_backward(sequences.float(), codebook, T_temp, L=L, k=k, V=V)
    return soft, None


def bcjr_forward_backward_fast(sequences, codebook, T_temp,
                               L=L_BITS, k=K_BITS, V=V_DIM,
                               preds=None, succs=None,
                               return_internals=False):
    """Drop-in for the no-checkpoint variant (src/bcjr/forward_backward_fast.py:75-...,
    selected by BCJR_FAST): the same node, so the same values and gradients."""
    return bcjr_forward_backward(sequences, codebook, T_temp, L=L, k=k, V=V, preds=preds, succs=succs,
                                 return_internals=return_internals)


def bcjr_forward_backward_monolithic_graphed(sequences, codebook, T_temp,
                                             preds=None, succs=None,
                                             return_internals=False,
                                             L=L_BITS, k=K_BITS, V=V_DIM):
    """Drop-in for src/bcjr/bcjr_monolithic_graph.py:41-81: (soft, None).  The
    reference captures its ~4N launches in a CUDA graph (BCJR_MONO_GRAPH=1); this
    node is one launch per direction with no host synchronisation, so a caller
    may capture it but gains nothing from it here."""
    return bcjr_forward_backward_monolithic(sequences, codebook, T_temp, L=L, k=k, V=V)


def reset_mono_graph_cache():
    """src/bcjr/bcjr_monolithic_graph.py:84-87.  No graphs are cached here."""


__all__ = [
    "L_BITS", "K_BITS", "V_DIM", "build_pred_succ_tables", "bcjr_forward_backward",
    "bcjr_forward_backward_monolithic", "BcjrFunction", "bcjr_forward_backward_fast",
    "bcjr_forward_backward_monolithic_graphed", "reset_mono_graph_cache",
]
