"""CPU oracle for the BCJR forward-backward path -- TEST INFRASTRUCTURE ONLY.

Only ``tests/``, ``__graft_entry__.smoke()`` and ``bench.py``'s ``cpu_baseline``
leg may import this package, and only to check results against (or as the
timed CPU baseline).  The product path under ``quant-2bit_amd/`` never imports it.

Contents
--------
``lib()``                 ctypes handle on ``oracle/_build/libbcjr_oracle.so``, the
                          C restatement (``bcjr_oracle.c``) of the reference's
                          eager BCJR node, gradient and Viterbi encoder.
``codebook / bcjr_forward / bcjr_backward / marginal_entropy / viterbi / viterbi_tailbiting / decode``
                          numpy-facing wrappers over the C restatement.
``naive_forward``         literal numpy restatement of the reference's eager
                          algorithm (gather over predecessor tables, then
                          logsumexp), src/bcjr/forward_backward.py:62-232.
``brute_force``           exhaustive path enumeration (tiny trellises only): exact
                          logZ, soft codeword and gradient (as the posterior
                          covariance of the codeword sequence), plus the
                          min-cost path.  Pins the recursions independently of
                          their form.
``viterbi_trace``         numpy restatement of the encoder's return_trace=True
                          lattices (src/viterbi/encode.py:250-307).
``pack_bits / unpack_bits``
                          2-bit (k*V-bit) LSB-first packing of per-step indices.
``fwht / rht / inverse_rht``
                          the random Hadamard transform of src/rht/transform.py.
``walk_states / dequant_unit / dequant_target``
                          walk replay and dequantization of saved targets
                          (src/quantize/lut_ft.py:59-79, src/quantize/serialize.py:56-107).

How each restatement is pinned (tests/test_oracle.py)
-----------------------------------------------------
bcjr_forward / bcjr_backward   brute-force path enumeration on tiny trellises (itself
                               checked by finite differences of log Z and soft), the
                               gather form ``naive_forward``, T -> inf / T -> 0 limits,
                               linearity of the gradient in g.
marginal_entropy               -sum P ln P of naive_forward's P; L ln 2 at T -> inf;
                               -> 0 at T -> 0 with a unique minimum.
viterbi_trace                  bit-exact against the float32 prefix costs of every
                               path (brute force: cum_t(s) is the smallest prefix cost
                               of the paths through s at t, and the backpointer the
                               lowest predecessor attaining it); its backtrace equals
                               the C encoder's walk and start.
viterbi / decode               the L=2 known answer of the reference's
                               test_viterbi.py:17-53, brute-force minimum-cost paths,
                               tie rules, the 1MAD Table-1 MSE band, round trips;
                               the constrained form against brute force over the
                               paths that meet the constraint (and its infeasible
                               cases), overlap_bits = 0 against the unconstrained.
viterbi_tailbiting             the wrap-around property of every walk and the MSE
                               gap of the reference's gate (test_viterbi.py:135-197).
codebook                       golden vectors written from src/codes/ref.py
                               (tests/golden/code_vectors.json).
pack_bits / unpack_bits        round trips and hand-checked byte layouts.
fwht / rht / inverse_rht       scipy.linalg.hadamard (Sylvester) matrix products,
                               bit-exact on integer inputs; rht . inverse_rht = I;
                               norm preservation.
walk_states / dequant_*        the C decode restatement (itself pinned above); the
                               sliding-window closed form of a state; tiles laid out
                               independently (matrix slices) reproduce a matrix
                               built from known walks; the scale's rounding against
                               exact rationals.
No function is parity unpinned.  What no check here can pin is the reference's
own float32 rounding of its eager torch ops (no fixtures of it exist).
"""
from __future__ import annotations

import ctypes
import itertools
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "_build", "libbcjr_oracle.so")
_lib = None

CODE_TABLE, CODE_1MAD, CODE_3INST, CODE_HYB = 0, 1, 2, 3


def build(force: bool = False) -> str:
    """Compile the C restatement with oracle/Makefile (gcc -O2 -fopenmp)."""
    if force or not os.path.exists(_LIB_PATH):
        subprocess.check_call(["make", "-s", "-C", _HERE], stdout=subprocess.DEVNULL)
    return _LIB_PATH


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        i32, i64, fp = ctypes.c_int, ctypes.c_int64, ctypes.c_void_p
        L.oracle_codebook.argtypes = [i32, i32, fp, i32, fp]
        L.oracle_bcjr_forward.argtypes = [i32, i32, i32, i64, i32, fp, fp, i32, fp, fp, fp, fp, i32]
        L.oracle_bcjr_backward.argtypes = [i32, i32, i32, i64, i32, fp, fp, i32, fp, fp, fp, fp, i32]
        L.oracle_viterbi.argtypes = [i32, i32, i32, i64, i32, fp, fp, fp, fp, fp, fp, fp, i32, fp, i32]
        L.oracle_decode.argtypes = [i32, i32, i32, i64, i32, fp, fp, fp, fp, fp]
        L.oracle_num_threads.argtypes = [i32]
        for name in ("oracle_codebook", "oracle_bcjr_forward", "oracle_bcjr_backward",
                     "oracle_viterbi", "oracle_decode", "oracle_num_threads"):
            getattr(L, name).restype = ctypes.c_int
        _lib = L
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data_as(ctypes.c_void_p)


def _f32(a):
    return np.ascontiguousarray(np.asarray(a, dtype=np.float32))


def _check(rc, what):
    if rc != 0:
        raise RuntimeError(f"oracle {what} failed with status {rc}")


def num_threads(n: int = 0) -> int:
    """Set (n > 0) and return the OpenMP thread count used by the C oracle."""
    return lib().oracle_num_threads(int(n))


def codebook(code: int, L: int, lut=None, Q: int = 9) -> np.ndarray:
    """(2^L, V) float32 codebook: 1MAD / 3INST (V=1) or HYB from a (2^Q, 2) LUT."""
    V = 2 if code == CODE_HYB else 1
    out = np.empty((1 << L, V), dtype=np.float32)
    lut_a = None if lut is None else _f32(lut)
    _check(lib().oracle_codebook(code, L, _ptr(lut_a), Q, _ptr(out)), "codebook")
    return out


def _temps(T, B):
    T = np.atleast_1d(np.asarray(T, dtype=np.float32))
    if T.size == 1:
        return _f32(T), 0
    assert T.size == B
    return _f32(T), 1


def bcjr_forward(seq, cb, T, L, KV, nthreads: int = 0):
    """soft (B,N,V) float32 and logZ (B,) float32, computed in float64."""
    seq = _f32(seq)
    cb = _f32(cb)
    B, N, V = seq.shape
    Ta, per = _temps(T, B)
    soft = np.empty_like(seq)
    logZ = np.empty((B,), dtype=np.float32)
    _check(lib().oracle_bcjr_forward(L, KV, V, B, N, _ptr(seq), _ptr(Ta), per, _ptr(cb),
                                      _ptr(soft), _ptr(logZ), None, nthreads), "forward")
    return soft, logZ


def marginal_entropy(seq, cb, T, L, KV, nthreads: int = 0):
    """H (B,N) float32: -sum_s P_t(s) ln P_t(s) in nats, computed in float64 --
    the per-(b, t) quantity entropy_diagnostic (src/bcjr/anneal.py:175-179)
    averages.  Pinned by naive_forward's P on small trellises and by the closed
    forms H = L ln 2 (uniform marginals at T -> inf) and H -> 0 (T -> 0, unique
    minimum)."""
    seq = _f32(seq)
    cb = _f32(cb)
    B, N, V = seq.shape
    Ta, per = _temps(T, B)
    soft = np.empty_like(seq)
    logZ = np.empty((B,), dtype=np.float32)
    H = np.empty((B, N), dtype=np.float32)
    _check(lib().oracle_bcjr_forward(L, KV, V, B, N, _ptr(seq), _ptr(Ta), per, _ptr(cb),
                                      _ptr(soft), _ptr(logZ), _ptr(H), nthreads), "forward")
    return H


def bcjr_backward(seq, cb, T, L, KV, g_soft, g_logZ=None, nthreads: int = 0):
    """d seq (B,N,V) for L = sum(g_soft * soft) + sum(g_logZ * logZ)."""
    seq = _f32(seq)
    cb = _f32(cb)
    g = _f32(g_soft)
    B, N, V = seq.shape
    Ta, per = _temps(T, B)
    gz = None if g_logZ is None else _f32(np.broadcast_to(np.asarray(g_logZ, np.float32), (B,)))
    d = np.empty_like(seq)
    _check(lib().oracle_bcjr_backward(L, KV, V, B, N, _ptr(seq), _ptr(Ta), per, _ptr(cb), _ptr(g),
                                       _ptr(gz), _ptr(d), nthreads), "backward")
    return d


def viterbi(seq, cb, L, KV, nthreads: int = 0, overlap=None, overlap_bits: int = 0):
    """Direct-form float32 Viterbi (src/viterbi/encode.py:250-307), batched.

    seq: (B, N, V).  Returns walk (B,N) int32, bitstream (B,N) int32,
    start_state (B,) int32, recon (B,N,V) float32, mse (B,) float32.
    With overlap ((B,) ints) the constraint of viterbi_encode_constrained_v
    (encode.py:328-389) applies with overlap_bits; start is -1 where no walk
    meets it (the reference raises).
    """
    seq = _f32(seq)
    cb = _f32(cb)
    B, N, V = seq.shape
    walk = np.empty((B, N), dtype=np.int32)
    bits = np.empty((B, N), dtype=np.int32)
    start = np.empty((B,), dtype=np.int32)
    recon = np.empty_like(seq)
    mse = np.empty((B,), dtype=np.float32)
    ov = None if overlap is None else np.ascontiguousarray(np.broadcast_to(
        np.asarray(overlap, dtype=np.int64), (B,)).astype(np.int32))
    _check(lib().oracle_viterbi(L, KV, V, B, N, _ptr(seq), _ptr(cb), _ptr(walk), _ptr(bits),
                                 _ptr(start), _ptr(recon), _ptr(mse), int(overlap_bits), _ptr(ov),
                                 nthreads), "viterbi")
    return walk, bits, start, recon, mse


def viterbi_tailbiting(seq, cb, L, k, V, nthreads: int = 0):
    """Tail-biting encoder, Algorithm 4 as viterbi_encode_tailbiting_v restates it
    (src/viterbi/encode.py:392-422; V = 1: :175-216), batched: rotate each
    sequence right by N//2 steps, encode it unconstrained, take the top L - kV
    bits of the rotated walk's state at step N//2 as the overlap, and encode the
    original under that constraint.  seq (B, N, V).  Returns walk, bitstream,
    start, recon, mse (as viterbi) and overlap (B,) int32."""
    seq = _f32(seq)
    B, N, _ = seq.shape
    kV = k * V
    walk_r, _, _, _, _ = viterbi(np.roll(seq, N // 2, axis=1), cb, L, kV, nthreads)
    overlap = (walk_r[:, N // 2] >> kV).astype(np.int32)
    return viterbi(seq, cb, L, kV, nthreads, overlap=overlap, overlap_bits=L - kV) + (overlap,)


def viterbi_trace(seq1, cb, L, KV):
    """The return_trace=True lattices of viterbi_encode_v for ONE sequence (N, V)
    (src/viterbi/encode.py:250-307), in numpy float32: trace[t, s] = cum_t(s),
    backptr[t, s] = the predecessor its minimum chose.  Predecessors of s are
    (p << (L - kV)) | (s >> kV), p ascending (encode.py:218-230); the first
    minimum wins; cum_{-1} = 0; the local cost is sum_v (c_v - w_v)^2 in float32."""
    x = np.asarray(seq1, np.float32)
    cb = np.asarray(cb, np.float32)
    S, R = 1 << L, 1 << KV
    states = np.arange(S, dtype=np.int64)
    pred = (np.arange(R, dtype=np.int64)[None, :] << (L - KV)) | (states[:, None] >> KV)  # (S, R)
    cum = np.zeros(S, np.float32)
    trace = np.empty((x.shape[0], S), np.float32)
    backptr = np.empty((x.shape[0], S), np.int32)
    for t in range(x.shape[0]):
        diff = cb - x[t][None, :]
        local = np.zeros(S, np.float32)
        for v in range(cb.shape[1]):
            local = local + diff[:, v] * diff[:, v]
        cand = cum[pred]                          # (S, R) costs of the predecessors
        first = np.argmin(cand, axis=1)           # lowest p among the minima
        cum = cand[states, first] + local
        trace[t] = cum
        backptr[t] = pred[states, first]
    return trace, backptr


def decode(bitstream, start, cb, L, KV):
    """Replay walks from (bitstream, start_state); returns walk and recon."""
    bits = np.ascontiguousarray(bitstream, dtype=np.int32)
    st = np.ascontiguousarray(start, dtype=np.int32)
    cb = _f32(cb)
    B, N = bits.shape
    V = cb.shape[1]
    walk = np.empty((B, N), dtype=np.int32)
    recon = np.empty((B, N, V), dtype=np.float32)
    _check(lib().oracle_decode(L, KV, V, B, N, _ptr(bits), _ptr(st), _ptr(cb), _ptr(walk),
                                _ptr(recon)), "decode")
    return walk, recon


# ---------------------------------------------------------------------------
# Literal restatement of the reference's eager algorithm (float64 numpy)
# ---------------------------------------------------------------------------

def pred_succ_tables(L, KV):
    """preds[s,p] = (p << (L-kV)) | (s >> kV); succs[s,c] = ((s << kV) | c) & mask.

    src/bcjr/forward_backward.py:62-86 (k*V passed as one bit count)."""
    S = 1 << L
    s = np.arange(S, dtype=np.int64)
    c = np.arange(1 << KV, dtype=np.int64)
    preds = (c[None, :] << (L - KV)) | (s >> KV)[:, None]
    succs = ((s[:, None] << KV) & (S - 1)) | c[None, :]
    return preds, succs


def _lse(x, axis):
    mx = np.max(x, axis=axis, keepdims=True)
    mx = np.where(np.isfinite(mx), mx, 0.0)
    return np.squeeze(mx, axis=axis) + np.log(np.sum(np.exp(x - mx), axis=axis))


def naive_forward(seq, cb, T, L, KV, return_internals=False):
    """Gather-over-predecessors BCJR exactly as forward_backward.py:89-232 (float64).

    Returns soft (B,N,V), logZ (B,) [, P, log_alpha, log_beta (B,N,S)].
    Memory is O(B*N*S): small trellises only.
    """
    seq = np.asarray(seq, dtype=np.float64)
    cb = np.asarray(cb, dtype=np.float64)
    B, N, V = seq.shape
    preds, succs = pred_succ_tables(L, KV)
    T = np.broadcast_to(np.asarray(T, dtype=np.float64).reshape(-1), (B,))
    cb_sq = (cb * cb).sum(-1)
    w_dot = np.einsum("bnv,sv->bns", seq, cb)
    w_sq = (seq * seq).sum(-1, keepdims=True)
    ll = -(cb_sq[None, None, :] - 2.0 * w_dot + w_sq) / T[:, None, None]
    la = np.zeros((B, N, 1 << L))
    prev = np.zeros((B, 1 << L))
    for t in range(N):
        prev = ll[:, t] + _lse(prev[:, preds], axis=-1)
        la[:, t] = prev
    lb = np.zeros((B, N, 1 << L))
    nxt = np.zeros((B, 1 << L))
    for t in range(N - 2, -1, -1):
        nxt = _lse(ll[:, t + 1][:, succs] + nxt[:, succs], axis=-1)
        lb[:, t] = nxt
    logZ = _lse(la[:, -1], axis=-1)
    P = np.exp(la + lb - logZ[:, None, None])
    soft = np.einsum("bns,sv->bnv", P, cb)
    if return_internals:
        return soft, logZ, P, la, lb
    return soft, logZ


# ---------------------------------------------------------------------------
# Brute force (exhaustive path enumeration, float64)
# ---------------------------------------------------------------------------

def enumerate_paths(L, KV, N):
    """All valid state paths (s_0..s_{N-1}) of the bitshift trellis, (P, N) int64."""
    S, R = 1 << L, 1 << KV
    paths = np.arange(S, dtype=np.int64)[:, None]
    for _ in range(N - 1):
        nxt = ((paths[:, -1:] << KV) & (S - 1))[:, :, None] | np.arange(R)[None, None, :]
        paths = np.concatenate(
            [np.repeat(paths, R, axis=0), nxt.reshape(-1, 1)], axis=1)
    return paths


def brute_force(seq1, cb, T, L, KV, g=None, g_logZ=0.0):
    """Exact quantities for ONE sequence (N,V) by enumerating every path.

    The start state s_{-1} is free (2^kV predecessors of s_0 each contribute
    weight 1), matching log_alpha_{-1} = 0 in forward_backward.py:143.
    Returns dict with logZ, soft (N,V), marg (N,S), and, when g (N,V) is given,
    grad (N,V) = (2/T) [Cov(F, c(s_t)) + g_logZ*(E c(s_t) - w_t)], the exact
    gradient of sum(g*soft) + g_logZ*logZ.  Also min-cost path data.
    """
    seq1 = np.asarray(seq1, dtype=np.float64)
    cb = np.asarray(cb, dtype=np.float64)
    N, V = seq1.shape
    paths = enumerate_paths(L, KV, N)
    cw = cb[paths]                                   # (P, N, V)
    cost = ((cw - seq1[None]) ** 2).sum(-1)          # (P, N)
    logw = -cost.sum(1) / T
    mx = logw.max()
    wts = np.exp(logw - mx)
    Zs = wts.sum()
    logZ = mx + np.log(Zs) + KV * np.log(2.0)
    pw = wts / Zs
    soft = np.einsum("p,pnv->nv", pw, cw)
    marg = np.zeros((N, 1 << L))
    for t in range(N):
        np.add.at(marg[t], paths[:, t], pw)
    out = {"logZ": logZ, "soft": soft, "marg": marg, "paths": paths, "cost": cost.sum(1)}
    if g is not None:
        g = np.asarray(g, dtype=np.float64)
        F = np.einsum("nv,pnv->p", g, cw)
        EF = (pw * F).sum()
        cov = np.einsum("p,pnv->nv", pw * (F - EF), cw)
        out["grad"] = (2.0 / T) * (cov + g_logZ * (soft - seq1))
    return out


def finite_difference_grad(seq1, cb, T, L, KV, g, g_logZ=0.0, h=1e-5):
    """Central differences of sum(g*soft)+g_logZ*logZ through brute_force (float64)."""
    seq1 = np.asarray(seq1, dtype=np.float64)
    grad = np.zeros_like(seq1)
    for idx in itertools.product(*[range(d) for d in seq1.shape]):
        vals = []
        for sgn in (+1, -1):
            x = seq1.copy()
            x[idx] += sgn * h
            r = brute_force(x, cb, T, L, KV)
            vals.append((np.asarray(g) * r["soft"]).sum() + g_logZ * r["logZ"])
        grad[idx] = (vals[0] - vals[1]) / (2 * h)
    return grad


# ---------------------------------------------------------------------------
# Bit packing of per-step indices
# ---------------------------------------------------------------------------

def pack_bits(bitstream, KV):
    """Pack (B, N) indices of KV bits each, LSB-first, into (B, ceil(N*KV/8)) uint8.

    Step t occupies bits [t*KV, (t+1)*KV) of the little-endian byte string.
    Only KV in {1, 2, 4, 8} is supported (indices never straddle a byte).
    """
    bits = np.asarray(bitstream, dtype=np.uint32)
    B, N = bits.shape
    assert KV in (1, 2, 4, 8)
    per = 8 // KV
    nbytes = (N * KV + 7) // 8
    out = np.zeros((B, nbytes), dtype=np.uint8)
    for t in range(N):
        out[:, t // per] |= ((bits[:, t] & ((1 << KV) - 1)) << ((t % per) * KV)).astype(np.uint8)
    return out


def unpack_bits(packed, N, KV):
    packed = np.asarray(packed, dtype=np.uint8)
    per = 8 // KV
    t = np.arange(N)
    return ((packed[:, t // per] >> ((t % per) * KV)) & ((1 << KV) - 1)).astype(np.int32)


# ---------------------------------------------------------------------------
# Random Hadamard transform (src/rht/transform.py)
# ---------------------------------------------------------------------------
def fwht(x):
    """Unscaled fast Walsh-Hadamard transform on the last axis in float32, with the
    butterflies of fwht_numpy (src/rht/transform.py:26-42): h = 1, 2, 4, ...,
    x[i] = a + b, x[i+h] = a - b.  Vectorised over the blocks of each stage; the
    arithmetic per element is the same."""
    x = np.array(x, dtype=np.float32, copy=True)
    n = x.shape[-1]
    assert n > 0 and n & (n - 1) == 0, n
    h = 1
    while h < n:
        v = x.reshape(x.shape[:-1] + (n // (2 * h), 2, h))
        a = v[..., 0, :].copy()
        b = v[..., 1, :].copy()
        v[..., 0, :] = a + b
        v[..., 1, :] = a - b
        h *= 2
    return x


def _rht_scale(W, m, n):
    # float32 result of dividing by sqrt(m*n) in float64, as the reference's
    # numpy path does (src/rht/transform.py:90-96)
    return (W.astype(np.float64) / np.sqrt(m * n)).astype(np.float32)


def rht(W, sign_l, sign_r):
    """H_m diag(sl) W diag(sr) H_n / sqrt(m n)  (src/rht/transform.py:65-96)."""
    W = np.asarray(W, dtype=np.float32)
    m, n = W.shape
    Wr = fwht(W * np.asarray(sign_r, np.float32)[None, :])
    Wl = fwht((Wr * np.asarray(sign_l, np.float32)[:, None]).T).T
    return _rht_scale(Wl, m, n)


def inverse_rht(W_tilde, sign_l, sign_r):
    """diag(sl) H_m W~ H_n diag(sr) / sqrt(m n)  (src/rht/transform.py:99-126)."""
    W = np.asarray(W_tilde, dtype=np.float32)
    m, n = W.shape
    Wr = fwht(W) * np.asarray(sign_r, np.float32)[None, :]
    Wl = fwht(Wr.T).T * np.asarray(sign_l, np.float32)[:, None]
    return _rht_scale(Wl, m, n)


# ---------------------------------------------------------------------------
# Dequantization of saved targets (src/quantize/serialize.py, lut_ft.py)
# ---------------------------------------------------------------------------
def walk_states(bitstreams, start_states, L, KV):
    """State walks s_t = ((s_{t-1} << KV) | b_t) & (2^L - 1) from s_{-1} = start,
    over any leading batch shape (src/quantize/lut_ft.py:59-79), int64."""
    bs = np.asarray(bitstreams, dtype=np.int64)
    s = np.asarray(start_states, dtype=np.int64).copy()
    mask = (1 << L) - 1
    walks = np.zeros_like(bs)
    for t in range(bs.shape[-1]):
        s = ((s << KV) | bs[..., t]) & mask
        walks[..., t] = s
    return walks


def dequant_unit(bitstreams, start_states, cb, shape, L, KV, Tx, Ty):
    """Unit-scale rotated-basis matrix (m, n) float64 of saved bitstreams
    (n_col_blocks, n_row_blocks, n_steps): column block j, row block i holds
    cb[walk] of tile (j, i) row-major (src/quantize/serialize.py:85-103)."""
    m, n = shape
    cb = np.asarray(cb, dtype=np.float32)
    walks = walk_states(bitstreams, start_states, L, KV)
    nc, nr, _ = walks.shape
    W = np.zeros((m, n), dtype=np.float64)
    for j in range(nc):
        W[:, j * Ty:(j + 1) * Ty] = cb[walks[j]].reshape(nr, Tx * Ty).astype(np.float64).reshape(m, Ty)
    return W


def dequant_target(bitstreams, start_states, cb, sign_l, sign_r, W_scale, shape, L, KV, Tx, Ty):
    """Weight in the original basis (src/quantize/serialize.py:56-107): the
    float64 product W_unit * W_scale, cast to float32 by the inverse RHT
    (src/rht/transform.py:99-126)."""
    W_tilde = dequant_unit(bitstreams, start_states, cb, shape, L, KV, Tx, Ty) * float(W_scale)
    return inverse_rht(W_tilde.astype(np.float32), np.asarray(sign_l, np.float32), np.asarray(sign_r, np.float32))
