"""Trellis codebooks built on the GPU by the engine's generators.

Drop-in for the codebook producers the quantizer uses: decode_1mad_batch /
decode_3inst_batch materialised over all states (src/codes/ref.py:33-41, :76-91)
and make_hyb_codebook_gpu (src/qat/ste.py:376-392).  Values are bit-identical
to the reference generators.  The returned (2^L, V) float32 tensor also records
its generator, so bcjr_forward_backward / the Viterbi encoder can hash c(s)
in-kernel instead of reading the table.
"""
from __future__ import annotations

import numpy as np
import torch

from . import ops
from .ops import CODE_1MAD, CODE_3INST, CODE_HYB


def _tag(cb: torch.Tensor, code: int, lut=None, Q: int = 9) -> torch.Tensor:
    cb._bcjr_code = code
    cb._bcjr_lut = lut
    cb._bcjr_Q = Q
    return cb


def make_1mad_codebook(L: int = 16, device="cuda") -> torch.Tensor:
    """(2^L, 1): ((byte sum of 34038481*s + 76625530) - 510) / 147.8."""
    return _tag(ops.codebook(CODE_1MAD, L, device), CODE_1MAD)


def make_3inst_codebook(L: int = 16, device="cuda") -> torch.Tensor:
    """(2^L, 1): fp16-pair sum of (89226354*s + 64248484) & 0x8FFF8FFF ^ fp16(0.922), / 1.2447."""
    return _tag(ops.codebook(CODE_3INST, L, device), CODE_3INST)


def make_hyb_codebook_gpu(lut_np, Q: int = 9, L_bits: int = 16, device="cuda") -> torch.Tensor:
    """(2^L, 2) from a (2^Q, 2) LUT: x = s*s + s, row (x >> (15-Q)) & (2^Q-1),
    second component negated when bit 15 of x is set (src/qat/ste.py:376-392)."""
    if torch.is_tensor(lut_np):
        lut = lut_np.detach().to(device=device, dtype=torch.float32).contiguous()
    else:
        lut = torch.from_numpy(np.ascontiguousarray(lut_np, dtype=np.float32)).to(device)
    if tuple(lut.shape) != (1 << Q, 2):
        raise AssertionError(f"LUT shape mismatch: {tuple(lut.shape)} != {(1 << Q, 2)}")
    return _tag(ops.codebook(CODE_HYB, L_bits, device, lut=lut, Q=Q), CODE_HYB, lut, Q)


def code_of(codebook: torch.Tensor) -> int:
    """Generator id recorded on a codebook (0 = plain table)."""
    return int(getattr(codebook, "_bcjr_code", 0))


__all__ = ["make_1mad_codebook", "make_3inst_codebook", "make_hyb_codebook_gpu", "code_of"]
