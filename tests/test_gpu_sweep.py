"""Seeded sweep over the engine's shape space against the oracle.

Beside the hand-picked cases of test_gpu_parity.py: shapes drawn from every
built (k, V) (k*V = 1, 2, 4, including k = 4 with V = 1), every trellis size
the ABI accepts for them, every codebook kind their V allows, odd sequence
lengths and batch sizes, Gaussian or heavy-tailed weights (Student-t, 5
degrees of freedom, unit variance), one temperature or one per sequence.
Each case checks the forward (soft, log Z), the gradient and the Viterbi
(walk, start state, reconstruction) at the bars of test_gpu_parity.py.
"""
import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu

SOFT_TOL, GRAD_TOL, LOGZ_TOL = 1e-4, 1e-3, 1e-5
SHAPES = [(1, 1), (2, 1), (1, 2), (2, 2), (4, 1)]  # (k, V)
LENGTHS = [1, 2, 3, 5, 7, 16, 33, 64, 100, 127, 200]


def _cases(n=64, seed=2026):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k, V = SHAPES[int(rng.integers(len(SHAPES)))]
        kV = k * V
        L = int(rng.integers(2 * kV, (11 if kV == 1 else 16) + 1))
        kinds = ["table"] + (["1mad", "3inst"] if V == 1 else ["hyb"])
        kind = kinds[int(rng.integers(len(kinds)))]
        N = int(rng.choice(LENGTHS))
        B = int(rng.integers(1, 7))
        if L >= 15:  # keep the float64 oracle to a few seconds per case
            B, N = min(B, 2), min(N, 128)
        T = round(float(np.exp(rng.uniform(np.log(0.04), np.log(2.0)))), 4)
        per_seq = bool(rng.integers(2)) and B > 1
        tails = bool(rng.integers(2))
        out.append((L, k, V, N, B, kind, T, per_seq, tails))
    return out


def _weights(rng, shape, tails):
    if tails:
        return (rng.standard_t(5, size=shape) / np.sqrt(5.0 / 3.0)).astype(np.float32)
    return rng.standard_normal(shape).astype(np.float32)


def _codebook(bcjr, kind, L, V, rng):
    if kind == "1mad":
        cb = bcjr.make_1mad_codebook(L, "cuda")
    elif kind == "3inst":
        cb = bcjr.make_3inst_codebook(L, "cuda")
    elif kind == "hyb":
        lut = rng.standard_normal((512, 2)).astype(np.float32)
        cb = bcjr.make_hyb_codebook_gpu(lut, Q=9, L_bits=L, device="cuda")
    else:
        cb = torch.tensor(rng.standard_normal((1 << L, V)).astype(np.float32), device="cuda")
    return cb, cb.cpu().numpy()


@pytest.mark.parametrize("L,k,V,N,B,kind,T,per_seq,tails", _cases())
def test_sweep_vs_oracle(bcjr_mod, oracle, L, k, V, N, B, kind, T, per_seq, tails):
    print(f"sweep L={L} k={k} V={V} N={N} B={B} {kind} T={T} per_seq={per_seq} tails={tails}", flush=True)
    from bcjr import bcjr_forward_backward, viterbi_encode_v_batched_hip
    rng = np.random.default_rng(L * 1000 + N * 10 + B)
    cb, cb_np = _codebook(bcjr_mod, kind, L, V, rng)
    seq = _weights(rng, (B, N, V), tails)
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    Ts = (T * np.exp(rng.uniform(-0.5, 0.5, B))).astype(np.float32) if per_seq else np.full(B, T, np.float32)
    T_arg = torch.tensor(Ts, device="cuda") if per_seq else T

    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, T_arg, L=L, k=k, V=V)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    soft_np, logZ_np, grad_np = soft.detach().cpu().numpy(), logZ.detach().cpu().numpy(), x.grad.cpu().numpy()
    for b in range(B):
        s_ref, z_ref = oracle.bcjr_forward(seq[b:b + 1], cb_np, float(Ts[b]), L, k * V)
        d_ref = oracle.bcjr_backward(seq[b:b + 1], cb_np, float(Ts[b]), L, k * V, g[b:b + 1])
        assert max_rel(soft_np[b:b + 1], s_ref) < SOFT_TOL, f"soft, sequence {b}"
        assert abs(float(logZ_np[b]) - float(z_ref[0])) <= LOGZ_TOL * max(1.0, abs(float(z_ref[0]))), \
            f"log Z, sequence {b}"
        assert max_rel(grad_np[b:b + 1], d_ref) < GRAD_TOL, f"gradient, sequence {b}"

    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(
        torch.tensor(seq.reshape(B, N * V), device="cuda"), cb, L=L, k=k, V=V, return_all=True)
    walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(seq, cb_np, L, k * V)
    assert np.array_equal(out["walk"].cpu().numpy(), walk_r)
    assert np.array_equal(bits.cpu().numpy(), bits_r)
    assert np.array_equal(start.cpu().numpy(), start_r)
    assert np.array_equal(recon.cpu().numpy(), recon_r.reshape(B, N * V))
