"""Test infrastructure: the reference's eager BCJR node restated in torch, run on
the CPU in float32 as the reference-semantics CPU baseline of bench.py (and
checked against the float64 C oracle in tests/test_oracle.py).  It is never
part of the product path.

It follows src/bcjr/forward_backward.py step for step:
  * emission by expansion, ll = -(|c|^2 - 2 <w, c> + |w|^2) / T (:89-103);
  * alpha: gather of the 2^kV predecessors, logsumexp, plus the emission,
    alpha_{-1} = 0, one autograd checkpoint per step when a gradient is wanted
    (:106-112, :122-154);
  * beta: gather of the successors' emission + beta, logsumexp,
    beta_{N-1} = 0, checkpointed likewise (:115-119, :157-187);
  * log Z = logsumexp of the last alpha, P = exp(alpha + beta - log Z),
    soft = P . codebook (:205-232);
  * the gradient is torch autograd through all of it.
"""
from __future__ import annotations

import torch
import torch.utils.checkpoint as ckpt


def trellis_tables(L: int, kV: int):
    """(preds, succs) int64 (2^L, 2^kV) of the bitshift trellis
    (src/bcjr/forward_backward.py:62-86)."""
    S, R = 1 << L, 1 << kV
    s = torch.arange(S, dtype=torch.int64)
    c = torch.arange(R, dtype=torch.int64)
    preds = (s >> kV).unsqueeze(1) | (c << (L - kV)).unsqueeze(0)
    succs = ((s << kV) & (S - 1)).unsqueeze(1) | c.unsqueeze(0)
    return preds, succs


def eager_bcjr(seq: torch.Tensor, codebook: torch.Tensor, T: float, L: int, kV: int, checkpoint: bool = True):
    """soft (B, N, V) and log Z (B,), differentiable with respect to seq."""
    preds, succs = trellis_tables(L, kV)
    B, N, V = seq.shape
    S = 1 << L
    T_t = torch.tensor(float(T), dtype=seq.dtype)
    cc = (codebook * codebook).sum(-1)
    ll = -(cc.view(1, 1, S) - 2.0 * torch.einsum("bnv,sv->bns", seq, codebook)
           + (seq * seq).sum(-1, keepdim=True)) / T_t
    use_ckpt = checkpoint and seq.requires_grad

    def a_step(prev, ll_t):
        return ll_t + torch.logsumexp(prev[:, preds], dim=-1)

    def b_step(nxt, ll_next):
        return torch.logsumexp(ll_next[:, succs] + nxt[:, succs], dim=-1)

    def run(fn, x, y):
        return ckpt.checkpoint(fn, x, y, use_reentrant=False) if use_ckpt else fn(x, y)

    alphas, cur = [], torch.zeros(B, S, dtype=seq.dtype)
    for t in range(N):
        cur = run(a_step, cur, ll[:, t])
        alphas.append(cur)
    betas, cur = [torch.zeros(B, S, dtype=seq.dtype)], None
    cur = betas[0]
    for t in range(N - 2, -1, -1):
        cur = run(b_step, cur, ll[:, t + 1])
        betas.append(cur)
    log_alpha = torch.stack(alphas, 1)
    log_beta = torch.stack(betas[::-1], 1)
    logZ = torch.logsumexp(log_alpha[:, -1], dim=-1)
    P = torch.exp(log_alpha + log_beta - logZ.view(B, 1, 1))
    soft = torch.einsum("bns,sv->bnv", P, codebook)
    return soft, logZ


def eager_step(seq, codebook, T, L, kV, g):
    """One QAT step of the eager node: forward, then the gradient of sum(g * soft).
    Returns (soft, logZ, d seq)."""
    x = seq.detach().clone().requires_grad_(True)
    soft, logZ = eager_bcjr(x, codebook, T, L, kV)
    soft.backward(g)
    return soft.detach(), logZ.detach(), x.grad
