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

import numpy as np
import torch

from . import _lib


def make_sign_vector(n, seed):
    """Random +-1 float32 vector of length n (src/rht/transform.py:58-62): the same
    generator and draw, so sign vectors saved with reference checkpoints match."""
    rng = np.random.default_rng(seed)
    return rng.choice([-1.0, 1.0], size=n).astype(np.float32)


# The transforms are the C++ operators bcjr::hadamard, bcjr::rht and
# bcjr::rht_batched (csrc/bcjr_torch.cpp, with their Meta kernels); their
# autograd formulas are registered here.
_ops = _lib.load_ops()


def _hadamard_setup(ctx, inputs, output):
    ctx.scale = inputs[1]


def _hadamard_backward(ctx, g):  # H is symmetric
    return _ops.hadamard(g.contiguous(), ctx.scale), None


torch.library.register_autograd("bcjr::hadamard", _hadamard_backward, setup_context=_hadamard_setup)


def _rht_setup(ctx, inputs, output):
    W, sign_l, sign_r, inverse = inputs
    ctx.save_for_backward(sign_l, sign_r)
    ctx.inverse = inverse


def _rht_backward(ctx, g):  # the adjoint of the transform is its inverse
    sign_l, sign_r = ctx.saved_tensors
    return _ops.rht(g.contiguous(), sign_l, sign_r, not ctx.inverse), None, None, None


def _rht_batched_backward(ctx, g):
    sign_l, sign_r = ctx.saved_tensors
    return _ops.rht_batched(g.contiguous(), sign_l, sign_r, not ctx.inverse), None, None, None


torch.library.register_autograd("bcjr::rht", _rht_backward, setup_context=_rht_setup)
torch.library.register_autograd("bcjr::rht_batched", _rht_batched_backward, setup_context=_rht_setup)


def hadamard_transform(x: torch.Tensor, scale: float = 1.0) -> torch.Tensor:
    """scale * H_n x along the last axis (unscaled Sylvester H_n, n a power of two): the
    fast_hadamard_transform call of src/qat/ste.py:113-135, with the butterflies of
    src/rht/transform.py:26-42 (fwht_numpy)."""
    if not x.is_cuda or x.dtype != torch.float32:
        raise AssertionError("hadamard_transform expects a float32 GPU tensor")
    return _lib.run_op(_ops.hadamard, x, float(scale))


def _check_rht_args(W, sign_l, sign_r):
    if W.dim() != 2 or not W.is_cuda or W.dtype != torch.float32:
        raise AssertionError(f"W must be a 2-D float32 GPU tensor; got {tuple(W.shape)} {W.dtype}")
    m, n = W.shape
    if tuple(sign_l.shape) != (m,) or tuple(sign_r.shape) != (n,):
        raise AssertionError(f"sign vectors must be ({m},) and ({n},); got {tuple(sign_l.shape)}, "
                             f"{tuple(sign_r.shape)}")


def _check_rht_batched_args(W, sign_l, sign_r):
    if W.dim() != 3 or not W.is_cuda or W.dtype != torch.float32:
        raise AssertionError(f"W must be a 3-D float32 GPU tensor; got {tuple(W.shape)} {W.dtype}")
    E, m, n = W.shape
    if tuple(sign_l.shape) != (E, m) or tuple(sign_r.shape) != (E, n):
        raise AssertionError(f"sign vectors must be ({E}, {m}) and ({E}, {n}); got {tuple(sign_l.shape)}, "
                             f"{tuple(sign_r.shape)}")


def _signs(v, like):
    return v.to(device=like.device, dtype=torch.float32)


def rht_op(W, sign_l, sign_r, inverse: bool) -> torch.Tensor:
    """The RHT of W (m, n), or its inverse (bcjr::rht over bcjr_rht)."""
    _check_rht_args(W, sign_l, sign_r)
    return _lib.run_op(_ops.rht, W, _signs(sign_l, W), _signs(sign_r, W), bool(inverse))


def rht_batched_op(W, sign_l, sign_r, inverse: bool) -> torch.Tensor:
    """The RHT (or its inverse) of each matrix of W (E, m, n) (bcjr::rht_batched
    over bcjr_rht_batched)."""
    _check_rht_batched_args(W, sign_l, sign_r)
    return _lib.run_op(_ops.rht_batched, W, _signs(sign_l, W), _signs(sign_r, W), bool(inverse))


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
