"""Hard straight-through trellis quantizer on the gfx950 Viterbi kernel.

Drop-in for src/qat/ste.py:160-357: quantize_forward_gpu_no_rht,
quantize_forward_gpu, quantize_forward_numpy, TrellisQuantSTE, TrellisQuantSTE_IP
and _replay_walks.
Data flow per weight: RHT (unless already rotated) -> RMS scale -> 16x16 tiles
-> Viterbi reconstruction -> untile -> rescale -> inverse RHT; the backward is
the identity (straight-through).  Every step runs on the GPU: the RHT on the FWHT
kernels, the Viterbi on bcjr_viterbi (the whole batch in one launch; its memory
is bounded by the engine's workspace, so no chunk loop is needed).

The reference fixes L = 16, k = 2, V = 2; here L and V follow the codebook's
shape (2^L, V) and k defaults to 2.  ptq_residual is the per-weight term of
measure_ptq_residual (src/bcjr/anneal.py:110-140).
"""
from __future__ import annotations

import numpy as np
import torch

from .quant import TX, TY, tile_for_viterbi, untile_from_viterbi
from .rht import apply_inverse_rht_gpu, apply_rht_gpu
from .viterbi import viterbi_encode_v_batched_hip

K_BITS = 2


def _lv(codebook):
    S, V = codebook.shape
    L = int(S).bit_length() - 1
    if S != 1 << L:
        raise AssertionError(f"codebook must have 2^L rows; got {S}")
    return L, V


def _rms(W):
    return W.pow(2).mean().sqrt().clamp(min=1e-30)


def _viterbi_recon_unit(W_unit, codebook, Tx, Ty, k):
    L, V = _lv(codebook)
    m, n = W_unit.shape
    seqs, info = tile_for_viterbi(W_unit.contiguous(), Tx, Ty)
    _, _, recons, _ = viterbi_encode_v_batched_hip(seqs.contiguous(), codebook, L=L, k=k, V=V)
    return untile_from_viterbi(recons, info, (m, n), Tx, Ty)


def quantize_forward_gpu_no_rht(W_rotated, codebook_gpu, Tx=TX, Ty=TY, k=K_BITS):
    """Hard-quantize a weight already in the rotated basis (src/qat/ste.py:160-180)."""
    W_scale = _rms(W_rotated)
    return _viterbi_recon_unit(W_rotated / W_scale, codebook_gpu, Tx, Ty, k) * W_scale


def quantize_forward_gpu(W_latent, sign_l_gpu, sign_r_gpu, codebook_gpu, Tx=TX, Ty=TY, k=K_BITS):
    """RHT -> hard quantize -> inverse RHT (src/qat/ste.py:183-212)."""
    W_tilde = apply_rht_gpu(W_latent, sign_l_gpu, sign_r_gpu)
    W_tilde_q = quantize_forward_gpu_no_rht(W_tilde, codebook_gpu, Tx, Ty, k)
    return apply_inverse_rht_gpu(W_tilde_q, sign_l_gpu, sign_r_gpu)


def quantize_forward_numpy(W_latent_np, sign_l_np, sign_r_np, codebook_gpu, Tx=TX, Ty=TY, k=K_BITS):
    """Numpy in, numpy out (src/qat/ste.py:213-267): RHT -> RMS scale -> tiles ->
    Viterbi -> untile -> rescale -> inverse RHT.  The transforms and the Viterbi
    run on the GPU kernels; the scale is the reference's numpy float32 RMS of the
    rotated weight.  Returns (W_q (m, n) float32, W_scale, walks (B, N) int64,
    bitstreams (B, N) int32, start_states (B,) int32)."""
    dev = codebook_gpu.device
    L, V = _lv(codebook_gpu)
    W = torch.from_numpy(np.ascontiguousarray(W_latent_np, dtype=np.float32)).to(dev)
    sl = torch.from_numpy(np.ascontiguousarray(sign_l_np, dtype=np.float32)).to(dev)
    sr = torch.from_numpy(np.ascontiguousarray(sign_r_np, dtype=np.float32)).to(dev)
    with torch.no_grad():
        W_tilde = apply_rht_gpu(W, sl, sr).cpu().numpy()
        W_scale = float(np.sqrt((W_tilde ** 2).mean()))
        if W_scale < 1e-30:
            W_scale = 1.0
        unit = torch.from_numpy(W_tilde / W_scale).to(dev)
        m, n = unit.shape
        seqs, info = tile_for_viterbi(unit, Tx, Ty)
        bits, start, recons, _ = viterbi_encode_v_batched_hip(seqs.contiguous(), codebook_gpu, L=L, k=k, V=V)
        W_tilde_q = untile_from_viterbi(recons, info, (m, n), Tx, Ty).cpu().numpy() * W_scale
        W_q = apply_inverse_rht_gpu(torch.from_numpy(W_tilde_q.astype(np.float32)).to(dev), sl, sr).cpu().numpy()
    bits_np, start_np = bits.cpu().numpy(), start.cpu().numpy()
    walks = replay_walks(bits_np.astype(np.int64), start_np.astype(np.int64), L=L, kV=k * V)
    return W_q.astype(np.float32), W_scale, walks, bits_np, start_np


def _f32_cuda(x, device):
    if isinstance(x, torch.Tensor):
        return x.detach().to(device=device, dtype=torch.float32)
    return torch.as_tensor(np.asarray(x, dtype=np.float32), device=device)


class TrellisQuantSTE(torch.autograd.Function):
    """W_q = TrellisQuantSTE.apply(W_latent, sign_l, sign_r, codebook_gpu); the
    gradient passes straight through (src/qat/ste.py:286-333).  W_latent must be a
    GPU tensor: there is no CPU path."""

    @staticmethod
    def forward(ctx, W_latent, sign_l, sign_r, codebook_gpu):
        if not W_latent.is_cuda:
            raise AssertionError("TrellisQuantSTE runs on the GPU; W_latent is on the CPU")
        dev = W_latent.device
        with torch.no_grad():
            W_q = quantize_forward_gpu(W_latent.detach().float(), _f32_cuda(sign_l, dev), _f32_cuda(sign_r, dev),
                                       codebook_gpu)
        return W_q.to(dtype=W_latent.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        return grad_output, None, None, None


class TrellisQuantSTE_IP(torch.autograd.Function):
    """Rotated-basis variant: W_q_rot = TrellisQuantSTE_IP.apply(W_rot, codebook_gpu)
    (src/qat/ste.py:336-357)."""

    @staticmethod
    def forward(ctx, W_latent_rotated, codebook_gpu):
        if not W_latent_rotated.is_cuda:
            raise AssertionError("IP mode requires CUDA")
        with torch.no_grad():
            W_q = quantize_forward_gpu_no_rht(W_latent_rotated.detach().float(), codebook_gpu)
        return W_q.to(dtype=W_latent_rotated.dtype)

    @staticmethod
    def backward(ctx, grad_output):
        return grad_output, None


def replay_walks(bitstreams, start_states, L=16, kV=4):
    """State walks from bitstreams and start states: s_t = ((s_{t-1} << kV) | b_t)
    & (2^L - 1), int64 (src/qat/ste.py:270-283; the reference fixes L=16, kV=4)."""
    b = np.asarray(bitstreams, dtype=np.int64)
    s = np.asarray(start_states, dtype=np.int64).copy()
    mask = (1 << L) - 1
    walks = np.zeros_like(b)
    for t in range(b.shape[1]):
        s = ((s << kV) | b[:, t]) & mask
        walks[:, t] = s
    return walks


def ptq_residual(W_latent, sign_l, sign_r, codebook_gpu):
    """(sum of squared unit-scale residuals, count) of one weight: the term that
    measure_ptq_residual (src/bcjr/anneal.py:110-140) accumulates over layers."""
    with torch.no_grad():
        dev = W_latent.device
        sl, sr = _f32_cuda(sign_l, dev), _f32_cuda(sign_r, dev)
        W_tilde = apply_rht_gpu(W_latent.float(), sl, sr)
        W_scale = _rms(W_tilde)
        W_q = TrellisQuantSTE.apply(W_latent, sl, sr, codebook_gpu)
        diff = W_tilde / W_scale - apply_rht_gpu(W_q.float(), sl, sr) / W_scale
        return float(diff.pow(2).sum()), diff.numel()


def _quantized_linears(layer):
    """The QuantizedLinear-like objects of a layer: anything exposing W_latent,
    sign_l, sign_r and codebook_gpu (the layer itself, its .modules(), or an
    iterable of them)."""
    attrs = ("W_latent", "sign_l", "sign_r", "codebook_gpu")
    if all(hasattr(layer, a) for a in attrs):
        return [layer]
    items = layer.modules() if hasattr(layer, "modules") else layer
    return [m for m in items if all(hasattr(m, a) for a in attrs)]


def measure_ptq_residual(qat_layer):
    """Mean squared unit-scale residual ||W~/s - RHT(W_q)/s||^2 over every
    quantized linear of a layer (src/bcjr/anneal.py:110-140): the natural T_0 of
    the annealing schedule."""
    accum, count = 0.0, 0
    for ql in _quantized_linears(qat_layer):
        ssq, n = ptq_residual(ql.W_latent, ql.sign_l, ql.sign_r, ql.codebook_gpu)
        accum += ssq
        count += n
    return accum / max(count, 1)


__all__ = ["quantize_forward_gpu_no_rht", "quantize_forward_gpu", "quantize_forward_numpy", "TrellisQuantSTE",
           "TrellisQuantSTE_IP", "replay_walks", "ptq_residual", "measure_ptq_residual"]
