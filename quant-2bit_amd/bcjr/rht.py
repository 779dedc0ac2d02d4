"""Random Hadamard transform (RHT) around the BCJR quantizer, on gfx950 kernels.

Drop-in for the GPU RHT of the reference:
  * hadamard_transform(x, scale)  -- fast_hadamard_transform.hadamard_transform,
    used by src/rht/transform.py:44-55 and src/qat/ste.py:113-135;
  * apply_rht_gpu / apply_inverse_rht_gpu (src/qat/ste.py:113-135), which equal
    apply_rht / apply_inverse_rht of src/rht/transform.py:65-126;
  * make_sign_vector (src/rht/transform.py:58-62);
  * apply_rht_batched / apply_inverse_rht_batched: the same transforms on a
    batch (E, m, n) with per-matrix sign vectors, in one launch pair (used by
    the expert-batched dispatch).

RHT(W) = H_m diag(sl) W diag(sr) H_n / sqrt(m n) is linear and its adjoint is
the inverse transform, so the autograd backward of each is the other one.
"""
from __future__ import annotations

import ctypes

import numpy as np
import torch

from . import _lib


def make_sign_vector(n, seed):
    """Random +-1 float32 vector of length n (src/rht/transform.py:58-62): the same
    generator and draw, so sign vectors saved with reference checkpoints match."""
    rng = np.random.default_rng(seed)
    return rng.choice([-1.0, 1.0], size=n).astype(np.float32)


def _stream(device):
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _hadamard(x: torch.Tensor, scale: float) -> torch.Tensor:
    if not x.is_cuda or x.dtype != torch.float32:
        raise AssertionError("hadamard_transform expects a float32 GPU tensor")
    n = x.shape[-1]
    xc = x.contiguous()
    out = torch.empty_like(xc)
    rows = xc.numel() // n if n else 0
    with torch.cuda.device(x.device):
        _lib.check(_lib.load().bcjr_hadamard(_lib.ptr(xc), _lib.ptr(out), rows, n, float(scale),
                                             _stream(x.device)), "bcjr_hadamard")
    return out


@torch.library.custom_op("bcjr::hadamard", mutates_args=())
def hadamard_op(x: torch.Tensor, scale: float) -> torch.Tensor:
    """scale * H_n x along the last axis (bcjr_hadamard)."""
    return _hadamard(x, scale)


@hadamard_op.register_fake
def _(x, scale):
    return torch.empty(x.shape, dtype=torch.float32, device=x.device)


def _hadamard_setup(ctx, inputs, output):
    ctx.scale = inputs[1]


def _hadamard_backward(ctx, g):  # H is symmetric
    return hadamard_op(g.contiguous(), ctx.scale), None


hadamard_op.register_autograd(_hadamard_backward, setup_context=_hadamard_setup)


def hadamard_transform(x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """scale * H_n x along the last axis (unscaled Sylvester H_n, n a power of two): the
    fast_hadamard_transform call of src/qat/ste.py:113-135, with the butterflies of
    src/rht/transform.py:26-42 (fwht_numpy)."""
    return hadamard_op(x, float(scale))


def _check_rht_args(W, sign_l, sign_r):
    if W.dim() != 2 or not W.is_cuda or W.dtype != torch.float32:
        raise AssertionError(f"W must be a 2-D float32 GPU tensor; got {tuple(W.shape)} {W.dtype}")
    m, n = W.shape
    if tuple(sign_l.shape) != (m,) or tuple(sign_r.shape) != (n,):
        raise AssertionError(f"sign vectors must be ({m},) and ({n},); got {tuple(sign_l.shape)}, "
                             f"{tuple(sign_r.shape)}")


def _rht(W, sign_l, sign_r, inverse: bool) -> torch.Tensor:
    _check_rht_args(W, sign_l, sign_r)
    m, n = W.shape
    Wc = W.detach().contiguous()
    sl = sign_l.detach().to(device=W.device, dtype=torch.float32).contiguous()
    sr = sign_r.detach().to(device=W.device, dtype=torch.float32).contiguous()
    out = torch.empty_like(Wc)
    with torch.cuda.device(W.device):
        _lib.check(_lib.load().bcjr_rht(_lib.ptr(Wc), _lib.ptr(out), m, n, _lib.ptr(sl), _lib.ptr(sr),
                                        1 if inverse else 0, _stream(W.device)), "bcjr_rht")
    return out


@torch.library.custom_op("bcjr::rht", mutates_args=())
def rht_op(W: torch.Tensor, sign_l: torch.Tensor, sign_r: torch.Tensor, inverse: bool) -> torch.Tensor:
    """The RHT of W (m, n), or its inverse (bcjr_rht)."""
    return _rht(W, sign_l, sign_r, inverse)


@rht_op.register_fake
def _(W, sign_l, sign_r, inverse):
    if W.dim() != 2 or tuple(sign_l.shape) != (W.shape[0],) or tuple(sign_r.shape) != (W.shape[1],):
        raise AssertionError(f"RHT of {tuple(W.shape)} with signs {tuple(sign_l.shape)}, {tuple(sign_r.shape)}")
    return torch.empty(W.shape, dtype=torch.float32, device=W.device)


def _rht_setup(ctx, inputs, output):
    W, sign_l, sign_r, inverse = inputs
    ctx.save_for_backward(sign_l, sign_r)
    ctx.inverse = inverse


def _rht_backward(ctx, g):  # the adjoint of the transform is its inverse
    sign_l, sign_r = ctx.saved_tensors
    return rht_op(g.contiguous(), sign_l, sign_r, not ctx.inverse), None, None, None


rht_op.register_autograd(_rht_backward, setup_context=_rht_setup)


def _rht_batched(W, sign_l, sign_r, inverse: bool) -> torch.Tensor:
    if W.dim() != 3 or not W.is_cuda or W.dtype != torch.float32:
        raise AssertionError(f"W must be a 3-D float32 GPU tensor; got {tuple(W.shape)} {W.dtype}")
    E, m, n = W.shape
    if tuple(sign_l.shape) != (E, m) or tuple(sign_r.shape) != (E, n):
        raise AssertionError(f"sign vectors must be ({E}, {m}) and ({E}, {n}); got {tuple(sign_l.shape)}, "
                             f"{tuple(sign_r.shape)}")
    Wc = W.detach().contiguous()
    sl = sign_l.detach().to(device=W.device, dtype=torch.float32).contiguous()
    sr = sign_r.detach().to(device=W.device, dtype=torch.float32).contiguous()
    out = torch.empty_like(Wc)
    with torch.cuda.device(W.device):
        _lib.check(_lib.load().bcjr_rht_batched(_lib.ptr(Wc), _lib.ptr(out), E, m, n, _lib.ptr(sl), _lib.ptr(sr),
                                                1 if inverse else 0, _stream(W.device)), "bcjr_rht_batched")
    return out


@torch.library.custom_op("bcjr::rht_batched", mutates_args=())
def rht_batched_op(W: torch.Tensor, sign_l: torch.Tensor, sign_r: torch.Tensor, inverse: bool) -> torch.Tensor:
    """The RHT (or its inverse) of each matrix of W (E, m, n) (bcjr_rht_batched)."""
    return _rht_batched(W, sign_l, sign_r, inverse)


@rht_batched_op.register_fake
def _(W, sign_l, sign_r, inverse):
    return torch.empty(W.shape, dtype=torch.float32, device=W.device)


def _rht_batched_backward(ctx, g):
    sign_l, sign_r = ctx.saved_tensors
    return rht_batched_op(g.contiguous(), sign_l, sign_r, not ctx.inverse), None, None, None


rht_batched_op.register_autograd(_rht_batched_backward, setup_context=_rht_setup)


def apply_rht_batched(W, sign_l, sign_r):
    """apply_rht_gpu (src/rht/transform.py:65-97) on each matrix of W (E, m, n),
    signs (E, m) and (E, n)."""
    return rht_batched_op(W, sign_l, sign_r, False)


def apply_inverse_rht_batched(W_tilde, sign_l, sign_r):
    """apply_inverse_rht_gpu (src/rht/transform.py:100-126) on each matrix of
    W_tilde (E, m, n)."""
    return rht_batched_op(W_tilde, sign_l, sign_r, True)


def _as_tensor(v, like):
    """Sign vector as a tensor (numpy arrays are accepted, as in the reference)."""
    return v if torch.is_tensor(v) else torch.as_tensor(np.asarray(v, dtype=np.float32), device=like.device)


def apply_rht_gpu(W, sign_l_gpu, sign_r_gpu):
    """W~ = H_m diag(sl) W diag(sr) H_n / sqrt(m n)  (src/qat/ste.py:113-126)."""
    return rht_op(W, _as_tensor(sign_l_gpu, W), _as_tensor(sign_r_gpu, W), False)


def apply_inverse_rht_gpu(W_tilde, sign_l_gpu, sign_r_gpu):
    """W = diag(sl) H_m W~ H_n diag(sr) / sqrt(m n)  (src/qat/ste.py:129-135)."""
    return rht_op(W_tilde, _as_tensor(sign_l_gpu, W_tilde), _as_tensor(sign_r_gpu, W_tilde), True)


__all__ = ["make_sign_vector", "hadamard_transform", "apply_rht_gpu", "apply_inverse_rht_gpu", "apply_rht_batched",
           "apply_inverse_rht_batched"]
