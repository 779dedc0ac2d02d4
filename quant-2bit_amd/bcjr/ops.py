"""Tensor-level wrappers over the engine's torch operators (torch.ops.bcjr.*,
registered in C++ by libbcjr_torch.so over the C ABI: outputs and workspace
from torch's caching allocator, the launch on the current stream).  These add
the reference's argument checks (AssertionError) and turn a failed C ABI call
into BcjrError.

Shapes follow the reference: sequences (B, N, V) float32, codebook (2^L, V),
bitstreams / walks (B, N) int32, start states (B,) int32.
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import _lib
from ._lib import CODE_1MAD, CODE_3INST, CODE_HYB, CODE_TABLE, OP_BACKWARD, OP_FORWARD, OP_VITERBI  # noqa: F401

_ops = _lib.load_ops()


@dataclass(frozen=True)
class Spec:
    """Static description of one trellis quantizer (everything but B, N, T)."""
    L: int
    k: int
    V: int
    code: int = CODE_TABLE
    Q: int = 9

    @property
    def kV(self) -> int:
        return self.k * self.V

    @property
    def S(self) -> int:
        return 1 << self.L

    def problem(self, B: int, N: int, t_per_seq: bool = False) -> _lib.Problem:
        return _lib.Problem(self.L, self.k, self.V, int(B), int(N), self.code, self.Q, int(bool(t_per_seq)))


def _temperature(T, B: int, device: torch.device):
    """float32 device tensor holding one T, or B of them; returns (tensor, per_seq).
    A python number is written by a fill kernel: no host-to-device copy, so the
    call can be captured into a graph."""
    if torch.is_tensor(T):
        Tt = T.detach().to(device=device, dtype=torch.float32).reshape(-1).contiguous()
    else:
        Tt = torch.full((1,), float(T), dtype=torch.float32, device=device)
    if Tt.numel() == 1:
        return Tt, False
    if Tt.numel() != B:
        raise AssertionError(f"T has {Tt.numel()} values; expected 1 or B={B}")
    return Tt, True


def _on(dev: torch.device, **tensors) -> None:
    """AssertionError unless every given tensor (None allowed) is on `dev`: the
    kernels dereference these pointers on that device."""
    for name, t in tensors.items():
        if t is not None and t.device != dev:
            raise AssertionError(f"{name} is on {t.device} but the launch runs on {dev}")


def _table(spec: Spec, codebook):
    """Pointer source for the codeword generator: table, HYB LUT or nothing."""
    if spec.code == CODE_TABLE:
        return codebook.detach().to(torch.float32).contiguous()
    if spec.code == CODE_HYB:
        return codebook.detach().to(torch.float32).contiguous()  # the (2^Q, 2) LUT
    return None


def _seq(seq: torch.Tensor) -> torch.Tensor:
    seq = seq.detach()
    return seq if seq.dtype == torch.float32 else seq.float()


def _soft(op, what, spec: Spec, seq, T, table):
    seq = _seq(seq)
    _on(seq.device, codebook_or_lut=table)
    Tt, _ = _temperature(T, seq.shape[0], seq.device)
    return _lib.run_op(op, seq, Tt, table, spec.L, spec.k, spec.V, spec.code, spec.Q)


def forward(spec: Spec, seq: torch.Tensor, T, table: torch.Tensor | None):
    """soft (B,N,V) float32 and logZ (B,) float32 (bcjr::forward)."""
    return _soft(_ops.forward, "bcjr_forward", spec, seq, T, table)


def forward_internals(spec: Spec, seq: torch.Tensor, T, table: torch.Tensor | None):
    """soft, logZ, P, log_alpha, log_beta; the last three are (B, N, 2^L) float32
    (bcjr::forward_internals)."""
    return _soft(_ops.forward_internals, "bcjr_forward_internals", spec, seq, T, table)


def forward_entropy(spec: Spec, seq: torch.Tensor, T, table: torch.Tensor | None):
    """soft, logZ and the marginal entropy H (B, N) in nats, H_t = -sum_s P log P
    (bcjr::forward_entropy)."""
    return _soft(_ops.forward_entropy, "bcjr_forward_entropy", spec, seq, T, table)


def backward(spec: Spec, seq: torch.Tensor, T, table, g_soft, g_logZ=None):
    """d seq (B,N,V) float32 of sum(g_soft*soft) + sum(g_logZ*logZ) (bcjr::backward)."""
    seq = _seq(seq)
    B, N, V = seq.shape
    _on(seq.device, codebook_or_lut=table, g_soft=g_soft)
    if g_soft is not None and tuple(g_soft.shape) != (B, N, V):
        raise AssertionError(f"g_soft must be {(B, N, V)}; got {tuple(g_soft.shape)}")
    Tt, _ = _temperature(T, B, seq.device)
    g = g_soft.detach() if g_soft is not None else torch.zeros_like(seq)
    gz = None if g_logZ is None else g_logZ.detach().to(device=seq.device, dtype=torch.float32)
    return _lib.run_op(_ops.backward, seq, Tt, table, g, gz, spec.L, spec.k, spec.V, spec.code, spec.Q)


def viterbi(spec: Spec, seq: torch.Tensor, table, want_packed: bool = True, overlap=None,
            overlap_bits: int | None = None):
    """Returns dict: walk, bitstream (B,N) int32; start (B,) int32; recon (B,N,V);
    mse (B,); packed (B, ceil(N*kV/8)) uint8 (if kV divides 8 and want_packed,
    else None) (bcjr::viterbi).  With overlap ((B,) int32 on the device) and
    overlap_bits, the tail-biting constraint of bcjr_viterbi_constrained
    applies; start is -1 for a sequence no walk satisfies."""
    seq = _seq(seq)
    _on(seq.device, codebook_or_lut=table)
    want = bool(want_packed and 8 % spec.kV == 0)
    ov = None
    if overlap is not None:
        ov = torch.as_tensor(overlap, dtype=torch.int32, device=seq.device).reshape(-1)
        if ov.numel() != seq.shape[0]:
            raise AssertionError(f"overlap has {ov.numel()} values for B={seq.shape[0]} sequences")
    walk, bits, start, recon, mse, packed = _lib.run_op(
        _ops.viterbi, seq, table, spec.L, spec.k, spec.V, spec.code, spec.Q, want, ov,
        int(overlap_bits or 0))
    return {"walk": walk, "bitstream": bits, "start": start, "recon": recon, "mse": mse,
            "packed": packed if want else None}


def decode(spec: Spec, start: torch.Tensor, table, bitstream=None, packed=None, N: int | None = None):
    """Replay walks; returns (walk (B,N) int32, recon (B,N,V) float32) (bcjr::decode)."""
    _on(start.device, codebook_or_lut=table, bitstream=bitstream, packed=packed)
    if bitstream is None and packed is None:
        raise AssertionError("need bitstream or packed")
    if bitstream is None and N is None:
        raise AssertionError("N is required with a packed bitstream")
    return _lib.run_op(_ops.decode, start, table, bitstream, packed, int(N or 0), spec.L, spec.k, spec.V,
                       spec.code, spec.Q, True)


def viterbi_trace(spec: Spec, x: torch.Tensor, table):
    """The full min-sum lattice of each sequence x (B, N, V): (trace (B, N, 2^L)
    float32 cumulative costs, backptr (B, N, 2^L) int32 chosen predecessor
    states), as viterbi_encode_v(..., return_trace=True) returns them for one
    sequence (src/viterbi/encode.py:250-307) (bcjr::viterbi_trace)."""
    _on(x.device, codebook_or_lut=table)
    if x.dim() != 3 or x.shape[2] != spec.V:
        raise AssertionError(f"sequences have V={x.shape[-1]}, spec V={spec.V}")
    return _lib.run_op(_ops.viterbi_trace, _seq(x), table, spec.L, spec.k, spec.V, spec.code, spec.Q)


def decode_walks(spec: Spec, start: torch.Tensor, bitstream: torch.Tensor) -> torch.Tensor:
    """Walks only: (B, N) int32 states replayed from start (B,) and a (B, N)
    bitstream; needs no codebook."""
    _on(start.device, bitstream=bitstream)
    walk, _ = _lib.run_op(_ops.decode, start, None, bitstream, None, 0, spec.L, spec.k, spec.V, spec.code,
                          spec.Q, False)
    return walk


BITS_U8, BITS_I32, BITS_PACKED = 0, 1, 2


def dequant(spec: Spec, start: torch.Tensor, table, m: int, n: int, Tx: int, Ty: int, scale: float,
            bitstream=None, packed=None) -> torch.Tensor:
    """(m, n) float32 matrix scale * c(walk) of Tx x Ty tiles, tile b = col_block *
    (m // Tx) + row_block, from a (B, N) uint8 / int32 bitstream or a packed one
    (bcjr::dequant)."""
    _on(start.device, codebook_or_lut=table, bitstream=bitstream, packed=packed)
    B = start.numel()
    N = (Tx * Ty) // spec.V
    if bitstream is not None:
        if bitstream.numel() != B * N:
            raise AssertionError(f"bitstream has {bitstream.numel()} steps, expected {B} tiles x {N}")
    elif packed is not None:
        nbytes = (N * spec.kV + 7) // 8
        if packed.numel() != B * nbytes:
            raise AssertionError(f"packed bitstream has {packed.numel()} bytes, expected {B} tiles x {nbytes}")
    else:
        raise AssertionError("need bitstream or packed")
    return _lib.run_op(_ops.dequant, start, table, bitstream, packed, int(m), int(n), int(Tx), int(Ty),
                       float(scale), spec.L, spec.k, spec.V, spec.code, spec.Q)


def codebook(code: int, L: int, device, lut: torch.Tensor | None = None, Q: int = 9) -> torch.Tensor:
    """(2^L, V) float32 codebook from a generator (1MAD, 3INST or HYB) (bcjr::codebook)."""
    device = torch.device(device)
    like = torch.empty(0, device=device)
    lut_t = None if lut is None else lut.detach().to(device=device, dtype=torch.float32)
    return _lib.run_op(_ops.codebook, like, lut_t, int(L), int(code), int(Q))


__all__ = ["Spec", "forward", "forward_internals", "forward_entropy", "backward", "viterbi", "decode",
           "decode_walks", "viterbi_trace", "dequant", "codebook", "CODE_TABLE", "CODE_1MAD",
           "CODE_3INST", "CODE_HYB"]
