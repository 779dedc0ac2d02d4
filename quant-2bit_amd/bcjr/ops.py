"""Tensor-level wrappers over the C ABI: allocate outputs and workspace with
torch's caching allocator, pass pointers and the current stream, raise on error.

Shapes follow the reference: sequences (B, N, V) float32, codebook (2^L, V),
bitstreams / walks (B, N) int32, start states (B,) int32.
"""
from __future__ import annotations

import ctypes
from dataclasses import dataclass

import torch

from . import _lib
from ._lib import CODE_1MAD, CODE_3INST, CODE_HYB, CODE_TABLE, OP_BACKWARD, OP_FORWARD, OP_VITERBI


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


def _stream(device: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(device).cuda_stream)


def _workspace(prob: _lib.Problem, op: int, device: torch.device) -> torch.Tensor:
    nbytes = ctypes.c_size_t(0)
    _lib.check(_lib.load().bcjr_workspace_bytes(ctypes.byref(prob), op, ctypes.byref(nbytes)),
               "bcjr_workspace_bytes")
    return torch.empty(max(int(nbytes.value), 1), dtype=torch.uint8, device=device)


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


def forward(spec: Spec, seq: torch.Tensor, T, table: torch.Tensor | None):
    """soft (B,N,V) float32 and logZ (B,) float32."""
    with torch.cuda.device(seq.device):
        seq = seq.detach().to(torch.float32).contiguous()
        B, N, V = seq.shape
        _on(seq.device, codebook_or_lut=table)
        Tt, per = _temperature(T, B, seq.device)
        soft = torch.empty_like(seq)
        logZ = torch.empty((B,), dtype=torch.float32, device=seq.device)
        if B == 0:
            return soft, logZ
        prob = spec.problem(B, N, per)
        ws = _workspace(prob, OP_FORWARD, seq.device)
        _lib.check(_lib.load().bcjr_forward(
            ctypes.byref(prob), _lib.ptr(seq), _lib.ptr(Tt), _lib.ptr(table), _lib.ptr(soft),
            _lib.ptr(logZ), _lib.ptr(ws), ws.numel(), _stream(seq.device)), "bcjr_forward")
        return soft, logZ


def forward_internals(spec: Spec, seq: torch.Tensor, T, table: torch.Tensor | None):
    """soft, logZ, P, log_alpha, log_beta; the last three are (B, N, 2^L) float32."""
    with torch.cuda.device(seq.device):
        seq = seq.detach().to(torch.float32).contiguous()
        B, N, V = seq.shape
        _on(seq.device, codebook_or_lut=table)
        Tt, per = _temperature(T, B, seq.device)
        soft = torch.empty_like(seq)
        logZ = torch.empty((B,), dtype=torch.float32, device=seq.device)
        P = torch.empty((B, N, spec.S), dtype=torch.float32, device=seq.device)
        la = torch.empty_like(P)
        lb = torch.empty_like(P)
        if B == 0:
            return soft, logZ, P, la, lb
        prob = spec.problem(B, N, per)
        ws = _workspace(prob, OP_FORWARD, seq.device)
        _lib.check(_lib.load().bcjr_forward_internals(
            ctypes.byref(prob), _lib.ptr(seq), _lib.ptr(Tt), _lib.ptr(table), _lib.ptr(soft),
            _lib.ptr(logZ), _lib.ptr(P), _lib.ptr(la), _lib.ptr(lb), _lib.ptr(ws), ws.numel(),
            _stream(seq.device)), "bcjr_forward_internals")
        return soft, logZ, P, la, lb


def forward_entropy(spec: Spec, seq: torch.Tensor, T, table: torch.Tensor | None):
    """soft, logZ and the marginal entropy H (B, N) in nats, H_t = -sum_s P log P."""
    with torch.cuda.device(seq.device):
        seq = seq.detach().to(torch.float32).contiguous()
        B, N, V = seq.shape
        _on(seq.device, codebook_or_lut=table)
        Tt, per = _temperature(T, B, seq.device)
        soft = torch.empty_like(seq)
        logZ = torch.empty((B,), dtype=torch.float32, device=seq.device)
        H = torch.empty((B, N), dtype=torch.float32, device=seq.device)
        if B == 0:
            return soft, logZ, H
        prob = spec.problem(B, N, per)
        ws = _workspace(prob, OP_FORWARD, seq.device)
        _lib.check(_lib.load().bcjr_forward_entropy(
            ctypes.byref(prob), _lib.ptr(seq), _lib.ptr(Tt), _lib.ptr(table), _lib.ptr(soft),
            _lib.ptr(logZ), _lib.ptr(H), _lib.ptr(ws), ws.numel(), _stream(seq.device)), "bcjr_forward_entropy")
        return soft, logZ, H


def backward(spec: Spec, seq: torch.Tensor, T, table, g_soft, g_logZ=None):
    """d seq (B,N,V) float32 of sum(g_soft*soft) + sum(g_logZ*logZ)."""
    with torch.cuda.device(seq.device):
        seq = seq.detach().to(torch.float32).contiguous()
        B, N, V = seq.shape
        _on(seq.device, codebook_or_lut=table, g_soft=g_soft)
        if g_soft is not None and tuple(g_soft.shape) != (B, N, V):
            raise AssertionError(f"g_soft must be {(B, N, V)}; got {tuple(g_soft.shape)}")
        Tt, per = _temperature(T, B, seq.device)
        g = g_soft.detach().to(torch.float32).contiguous() if g_soft is not None else torch.zeros_like(seq)
        gz = None
        if g_logZ is not None:
            gz = g_logZ.detach().to(device=seq.device, dtype=torch.float32).reshape(-1).expand(B).contiguous()
        d = torch.empty_like(seq)
        if B == 0:
            return d
        prob = spec.problem(B, N, per)
        ws = _workspace(prob, OP_BACKWARD, seq.device)
        _lib.check(_lib.load().bcjr_backward(
            ctypes.byref(prob), _lib.ptr(seq), _lib.ptr(Tt), _lib.ptr(table), None, _lib.ptr(g),
            _lib.ptr(gz), _lib.ptr(d), _lib.ptr(ws), ws.numel(), _stream(seq.device)), "bcjr_backward")
        return d


def viterbi(spec: Spec, seq: torch.Tensor, table, want_packed: bool = True, overlap=None,
            overlap_bits: int | None = None):
    """Returns dict: walk, bitstream (B,N) int32; start (B,) int32; recon (B,N,V);
    mse (B,); packed (B, ceil(N*kV/8)) uint8 (if kV divides 8 and want_packed).
    With overlap ((B,) int32 on the device) and overlap_bits, the tail-biting
    constraint of bcjr_viterbi_constrained applies; start is -1 for a sequence
    no walk satisfies."""
    with torch.cuda.device(seq.device):
        seq = seq.detach().to(torch.float32).contiguous()
        B, N, V = seq.shape
        dev = seq.device
        _on(dev, codebook_or_lut=table)
        out = {
            "walk": torch.empty((B, N), dtype=torch.int32, device=dev),
            "bitstream": torch.empty((B, N), dtype=torch.int32, device=dev),
            "start": torch.empty((B,), dtype=torch.int32, device=dev),
            "recon": torch.empty_like(seq),
            "mse": torch.empty((B,), dtype=torch.float32, device=dev),
        }
        packed = None
        if want_packed and 8 % spec.kV == 0:
            packed = torch.empty((B, (N * spec.kV + 7) // 8), dtype=torch.uint8, device=dev)
        out["packed"] = packed
        if B == 0:
            return out
        prob = spec.problem(B, N)
        ws = _workspace(prob, OP_VITERBI, dev)
        if overlap is None:
            _lib.check(_lib.load().bcjr_viterbi(
                ctypes.byref(prob), _lib.ptr(seq), _lib.ptr(table), _lib.ptr(out["walk"]),
                _lib.ptr(out["bitstream"]), _lib.ptr(out["start"]), _lib.ptr(out["recon"]),
                _lib.ptr(out["mse"]), _lib.ptr(packed), _lib.ptr(ws), ws.numel(), _stream(dev)),
                "bcjr_viterbi")
        else:
            ov = torch.as_tensor(overlap, dtype=torch.int32, device=dev).reshape(-1).contiguous()
            if ov.numel() != B:
                raise AssertionError(f"overlap has {ov.numel()} values for B={B} sequences")
            _lib.check(_lib.load().bcjr_viterbi_constrained(
                ctypes.byref(prob), _lib.ptr(seq), _lib.ptr(table), int(overlap_bits), _lib.ptr(ov),
                _lib.ptr(out["walk"]), _lib.ptr(out["bitstream"]), _lib.ptr(out["start"]),
                _lib.ptr(out["recon"]), _lib.ptr(out["mse"]), _lib.ptr(packed), _lib.ptr(ws), ws.numel(),
                _stream(dev)), "bcjr_viterbi_constrained")
        return out


def decode(spec: Spec, start: torch.Tensor, table, bitstream=None, packed=None, N: int | None = None):
    """Replay walks; returns (walk (B,N) int32, recon (B,N,V) float32)."""
    dev = start.device
    _on(dev, codebook_or_lut=table, bitstream=bitstream, packed=packed)
    with torch.cuda.device(dev):
        start = start.to(torch.int32).contiguous()
        B = start.shape[0]
        if bitstream is not None:
            bitstream = bitstream.to(torch.int32).contiguous()
            N = bitstream.shape[1]
        elif packed is not None:
            packed = packed.to(torch.uint8).contiguous()
            if N is None:
                raise AssertionError("N is required with a packed bitstream")
        else:
            raise AssertionError("need bitstream or packed")
        walk = torch.empty((B, N), dtype=torch.int32, device=dev)
        recon = torch.empty((B, N, spec.V), dtype=torch.float32, device=dev)
        if B == 0:
            return walk, recon
        prob = spec.problem(B, N)
        _lib.check(_lib.load().bcjr_decode(
            ctypes.byref(prob), _lib.ptr(bitstream), _lib.ptr(packed), _lib.ptr(start),
            _lib.ptr(table), _lib.ptr(walk), _lib.ptr(recon), _stream(dev)), "bcjr_decode")
        return walk, recon


def viterbi_trace(spec: Spec, x: torch.Tensor, table):
    """The full min-sum lattice of each sequence x (B, N, V): (trace (B, N, 2^L)
    float32 cumulative costs, backptr (B, N, 2^L) int32 chosen predecessor
    states), as viterbi_encode_v(..., return_trace=True) returns them for one
    sequence (src/viterbi/encode.py:250-307)."""
    dev = x.device
    _on(dev, codebook_or_lut=table)
    with torch.cuda.device(dev):
        x = x.to(torch.float32).contiguous()
        B, N, V = x.shape
        if V != spec.V:
            raise AssertionError(f"sequences have V={V}, spec V={spec.V}")
        S = 1 << spec.L
        trace = torch.empty((B, N, S), dtype=torch.float32, device=dev)
        backptr = torch.empty((B, N, S), dtype=torch.int32, device=dev)
        if B == 0 or N == 0:
            return trace, backptr
        prob = spec.problem(B, N)
        _lib.check(_lib.load().bcjr_viterbi_trace(
            ctypes.byref(prob), _lib.ptr(x), _lib.ptr(table), _lib.ptr(trace), _lib.ptr(backptr),
            _stream(dev)), "bcjr_viterbi_trace")
        return trace, backptr


def decode_walks(spec: Spec, start: torch.Tensor, bitstream: torch.Tensor) -> torch.Tensor:
    """Walks only: (B, N) int32 states replayed from start (B,) and a (B, N)
    bitstream; needs no codebook."""
    dev = start.device
    _on(dev, bitstream=bitstream)
    with torch.cuda.device(dev):
        start = start.to(torch.int32).contiguous()
        bitstream = bitstream.to(torch.int32).contiguous()
        B, N = bitstream.shape
        walk = torch.empty((B, N), dtype=torch.int32, device=dev)
        if B == 0 or N == 0:
            return walk
        prob = spec.problem(B, N)
        _lib.check(_lib.load().bcjr_decode(
            ctypes.byref(prob), _lib.ptr(bitstream), None, _lib.ptr(start), None, _lib.ptr(walk), None,
            _stream(dev)), "bcjr_decode")
        return walk


BITS_U8, BITS_I32, BITS_PACKED = 0, 1, 2


def dequant(spec: Spec, start: torch.Tensor, table, m: int, n: int, Tx: int, Ty: int, scale: float,
            bitstream=None, packed=None) -> torch.Tensor:
    """(m, n) float32 matrix scale * c(walk) of Tx x Ty tiles, tile b = col_block *
    (m // Tx) + row_block, from a (B, N) uint8 / int32 bitstream or a packed one."""
    dev = start.device
    _on(dev, codebook_or_lut=table, bitstream=bitstream, packed=packed)
    with torch.cuda.device(dev):
        start = start.reshape(-1).to(torch.int32).contiguous()
        B = start.shape[0]
        N = (Tx * Ty) // spec.V
        if bitstream is not None:
            if bitstream.numel() != B * N:
                raise AssertionError(f"bitstream has {bitstream.numel()} steps, expected {B} tiles x {N}")
            fmt = BITS_U8 if bitstream.dtype == torch.uint8 else BITS_I32
            bits = bitstream.reshape(B, N)
            bits = bits.contiguous() if fmt == BITS_U8 else bits.to(torch.int32).contiguous()
        elif packed is not None:
            fmt = BITS_PACKED
            nbytes = (N * spec.kV + 7) // 8
            if packed.numel() != B * nbytes:
                raise AssertionError(f"packed bitstream has {packed.numel()} bytes, expected {B} tiles x {nbytes}")
            bits = packed.reshape(B, nbytes).to(torch.uint8).contiguous()
        else:
            raise AssertionError("need bitstream or packed")
        out = torch.empty((m, n), dtype=torch.float32, device=dev)
        prob = spec.problem(B, N)
        _lib.check(_lib.load().bcjr_dequant(
            ctypes.byref(prob), _lib.ptr(bits), fmt, _lib.ptr(start), _lib.ptr(table), m, n, Tx, Ty,
            float(scale), _lib.ptr(out), _stream(dev)), "bcjr_dequant")
        return out


def codebook(code: int, L: int, device, lut: torch.Tensor | None = None, Q: int = 9) -> torch.Tensor:
    """(2^L, V) float32 codebook from a generator (1MAD, 3INST or HYB)."""
    device = torch.device(device)
    V = 2 if code == CODE_HYB else 1
    out = torch.empty((1 << L, V), dtype=torch.float32, device=device)
    with torch.cuda.device(device):
        lut_t = None if lut is None else lut.detach().to(device=device, dtype=torch.float32).contiguous()
        prob = _lib.Problem(L, 2, V, 0, 1, code, Q, 0)
        _lib.check(_lib.load().bcjr_codebook(ctypes.byref(prob), _lib.ptr(lut_t), _lib.ptr(out),
                                             _stream(device)), "bcjr_codebook")
    return out


__all__ = ["Spec", "forward", "forward_internals", "backward", "viterbi", "decode", "decode_walks", "dequant",
           "codebook", "CODE_TABLE", "CODE_1MAD", "CODE_3INST", "CODE_HYB"]
