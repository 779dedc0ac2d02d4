"""BCJR forward-backward node on the bitshift trellis, backed by gfx950 HIP kernels.

Drop-in for src/bcjr/forward_backward.py (bcjr_forward_backward,
build_pred_succ_tables, L_BITS/K_BITS/V_DIM) and src/bcjr/bcjr_monolithic.py
(bcjr_forward_backward_monolithic): same call signatures, tensor layouts,
return values and assertion behaviour.  The whole forward (alpha and beta
recursions, marginals, soft codeword, log Z) is one kernel launch, and the
backward is one more; autograd saves only the inputs.

The node is the registered torch operator bcjr::node (torch.library.custom_op,
with a fake implementation and an autograd formula whose backward is
bcjr::node_backward), so torch.compile traces through it without a graph break
(the reference compiles its node: src/bcjr/forward_backward_fast.py:33-44,
src/tripwires/test_bcjr_compile.py:28-84).  Inside, it resolves the codebook
and calls the C++ operators bcjr::forward / bcjr::backward (libbcjr_torch.so,
TORCH_LIBRARY over the C ABI).

Trellis (forward_backward.py:1-45): S = 2^L states, kV = k*V bits per step,
next = ((s << kV) | c) & (S-1); emission ll_t(s) = -||c(s) - w_t||^2 / T;
log_alpha_{-1} = 0 (free start), log_beta_{N-1} = 0 (free end).

Codebooks.  `codebook` is the (2^L, V) float32 table, as in the reference.  The
kernels hash c(s) in-kernel for the 1MAD / 3INST codebooks and read a staged LUT
for HYB ones, whether the table was made by bcjr.codes or recognised by content
(bcjr.codes.resolve_codebook); any other table is read as a table.

Temperature.  A python float, a 0-d / (1,) tensor, or a (B,) tensor (one value
per sequence).  A python float becomes a one-element device tensor through a
fill kernel, so the node makes no host-to-device copy and can be captured.  T
must be finite and > 0: a sequence whose T is not, or whose weights (or, in the
backward, upstream gradients) are not all finite, gets NaN outputs.
"""
from __future__ import annotations

from typing import Optional

import torch
from torch import Tensor

from . import ops
from .codes import resolve_codebook

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


def _check_args(sequences, codebook, L, k, V, preds, succs):
    # Same conditions as forward_backward.py:206-207, plus table shapes and devices.
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
    if codebook.device != sequences.device:
        raise AssertionError(f"codebook is on {codebook.device} but the sequences are on {sequences.device}")


def temperature_tensor(T, device: torch.device) -> Tensor:
    """T as a float32 device tensor: (1,) for one value, (B,) for one per sequence.
    A python number is written by a fill kernel (no host-to-device copy)."""
    if torch.is_tensor(T):
        t = T.detach()
        if t.device != device and t.numel() == 1 and t.device.type == "cpu":
            return torch.full((1,), float(t), dtype=torch.float32, device=device)
        return t.to(device=device, dtype=torch.float32).reshape(-1)
    return torch.full((1,), float(T), dtype=torch.float32, device=device)


def _check_T(T: Tensor, B: int):
    if T.numel() not in (1, B):
        raise AssertionError(f"T has {T.numel()} values; expected 1 or B={B}")


# ---------------------------------------------------------------------------
# Registered operators
# ---------------------------------------------------------------------------

@torch.library.custom_op("bcjr::node", mutates_args=())
def bcjr_forward_op(sequences: Tensor, codebook: Tensor, T: Tensor, L: int, k: int,
                    V: int) -> tuple[Tensor, Tensor]:
    """soft (B, N, V) and log Z (B,), float32: the node's forward on a (2^L, V)
    codebook (resolved here, then bcjr::forward)."""
    _check_T(T, sequences.shape[0])
    spec, table = resolve_codebook(codebook, L, k, V, sequences.device)
    return ops.forward(spec, sequences, T, table)


@bcjr_forward_op.register_fake
def _(sequences, codebook, T, L, k, V):
    B, N, Vs = sequences.shape
    return (sequences.new_empty((B, N, Vs), dtype=torch.float32),
            sequences.new_empty((B,), dtype=torch.float32))


@torch.library.custom_op("bcjr::node_backward", mutates_args=())
def bcjr_backward_op(sequences: Tensor, codebook: Tensor, T: Tensor, g_soft: Tensor,
                     g_logZ: Optional[Tensor], L: int, k: int, V: int) -> Tensor:
    """d sequences (B, N, V) float32 of sum(g_soft * soft) + sum(g_logZ * logZ)
    (the codebook resolved, then bcjr::backward)."""
    _check_T(T, sequences.shape[0])
    spec, table = resolve_codebook(codebook, L, k, V, sequences.device)
    return ops.backward(spec, sequences, T, table, g_soft, g_logZ)


@bcjr_backward_op.register_fake
def _(sequences, codebook, T, g_soft, g_logZ, L, k, V):
    return torch.empty_like(sequences, dtype=torch.float32)


def _fwd_setup(ctx, inputs, output):
    sequences, codebook, T, L, k, V = inputs
    ctx.save_for_backward(sequences, codebook, T)
    ctx.lkv = (L, k, V)


def _fwd_backward(ctx, g_soft, g_logZ):
    sequences, codebook, T = ctx.saved_tensors
    L, k, V = ctx.lkv
    if g_soft is None:
        g_soft = torch.zeros_like(sequences)
    d = bcjr_backward_op(sequences, codebook, T, g_soft.contiguous(), g_logZ, L, k, V)
    return d, None, None, None, None, None


bcjr_forward_op.register_autograd(_fwd_backward, setup_context=_fwd_setup)


class BcjrInternalsFunction(torch.autograd.Function):
    """return_internals=True: soft and log Z on the autograd graph (the
    reference's eager node returns them differentiable,
    src/bcjr/forward_backward.py:220-231); P, log alpha and log beta are
    returned without gradient.  The backward is the node's backward."""

    @staticmethod
    def forward(ctx, sequences, codebook, T, L, k, V):
        spec, table = resolve_codebook(codebook, L, k, V, sequences.device)
        soft, logZ, P, la, lb = ops.forward_internals(spec, sequences, T, table)
        ctx.save_for_backward(sequences, codebook, T)
        ctx.lkv = (L, k, V)
        ctx.mark_non_differentiable(P, la, lb)
        return soft, logZ, P, la, lb

    @staticmethod
    def backward(ctx, g_soft, g_logZ, gP, gla, glb):
        sequences, codebook, T = ctx.saved_tensors
        L, k, V = ctx.lkv
        if g_soft is None:
            g_soft = torch.zeros_like(sequences)
        d = bcjr_backward_op(sequences, codebook, T, g_soft.contiguous(), g_logZ, L, k, V)
        return d, None, None, None, None, None


class BcjrFunction:
    """The node as one autograd function (forward = bcjr::node, backward =
    bcjr::node_backward): BcjrFunction.apply(sequences, codebook, T, L, k, V)."""

    @staticmethod
    def apply(sequences, codebook, T, L, k, V):
        return bcjr_forward_op(sequences, codebook, T, L, k, V)


def bcjr_forward_backward(sequences, codebook, T_temp,
                          L=L_BITS, k=K_BITS, V=V_DIM,
                          preds=None, succs=None, return_internals=False):
    """Full BCJR forward-backward (forward_backward.py:190-232).

    sequences: (B, N, V) float, requires_grad allowed.
    codebook:  (2^L, V) float32 on the sequences' device (no gradient).
    T_temp:    temperature > 0: python float, 0-d tensor, or (B,) tensor (one
               per sequence, for batching several tensors in one call).

    Returns (soft (B,N,V), log_Z (B,)), or with return_internals
    (soft, log_Z, P, log_alpha, log_beta) with the last three (B, N, 2^L).
    soft and log_Z are differentiable with respect to sequences in both forms.
    """
    _check_args(sequences, codebook, L, k, V, preds, succs)
    dt = sequences.dtype
    seq = sequences if dt == torch.float32 else sequences.float()
    T = temperature_tensor(T_temp, sequences.device)
    if return_internals:
        soft, logZ, P, la, lb = BcjrInternalsFunction.apply(seq.contiguous(), codebook, T, L, k, V)
        return soft.to(dt), logZ.to(dt), P, la, lb
    soft, logZ = bcjr_forward_op(seq.contiguous(), codebook, T, L, k, V)
    return soft.to(dt), logZ.to(dt)


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
    "bcjr_forward_backward_monolithic", "BcjrFunction", "BcjrInternalsFunction", "bcjr_forward_backward_fast",
    "bcjr_forward_backward_monolithic_graphed", "reset_mono_graph_cache", "bcjr_forward_op",
    "bcjr_backward_op", "temperature_tensor",
]
