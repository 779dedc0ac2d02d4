"""GPU parity tests: HIP kernels (through the C ABI) vs the CPU oracle.

Bars (from the reference's parity gates and the engine contract):
  soft codeword  max|d|/max|ref| <= 1e-4   (test_bcjr_triton_parity.py:28 step gate)
  gradients      max|d|/max|ref| <= 1e-3   (test_bcjr_monolithic_parity.py:43,53)
  log Z          |d| <= 1e-5 * max|log Z|
  Viterbi walk / bitstream / start state / recon: bit-exact.
"""
import hashlib
import json
import os

import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "code_vectors.json")
SOFT_TOL, GRAD_TOL, LOGZ_TOL = 1e-4, 1e-3, 1e-5


def _say(msg):
    print(msg, flush=True)


def _rng_case(seed, B, N, V, L, table=True):
    rng = np.random.default_rng(seed)
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32) if table else None
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    return seq, cb, g


def _codebook(bcjr, oracle, kind, L, dev):
    """Returns (tagged device codebook, numpy table) for kind in table/1mad/3inst/hyb."""
    if kind == "1mad":
        cb = bcjr.make_1mad_codebook(L, dev)
    elif kind == "3inst":
        cb = bcjr.make_3inst_codebook(L, dev)
    elif kind == "hyb":
        lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
        cb = bcjr.make_hyb_codebook_gpu(lut, Q=9, L_bits=L, device=dev)
    else:
        raise ValueError(kind)
    return cb, cb.cpu().numpy()


# --------------------------------------------------------------------------
# codebook generators
# --------------------------------------------------------------------------

@pytest.mark.parametrize("name", ["1mad", "3inst", "hyb"])
def test_codebook_bit_exact(bcjr_mod, oracle, name):
    _say(f"codebook {name}")
    g = json.load(open(GOLDEN))
    cb, cb_np = _codebook(bcjr_mod, oracle, name, g["L"], "cuda")
    torch.cuda.synchronize()
    assert hashlib.sha256(np.ascontiguousarray(cb_np).tobytes()).hexdigest() == g["codes"][name]["sha256_f32"]


# --------------------------------------------------------------------------
# soft forward / backward
# --------------------------------------------------------------------------

TINY = [  # (L, k, V, N, T) against exhaustive enumeration
    (4, 2, 1, 5, 0.7), (4, 1, 2, 4, 1.3), (6, 2, 1, 6, 0.05), (8, 2, 2, 3, 1.0), (3, 1, 1, 5, 0.2),
]


@pytest.mark.parametrize("L,k,V,N,T", TINY)
def test_forward_backward_tiny_vs_brute_force(bcjr_mod, oracle, L, k, V, N, T):
    _say(f"tiny L={L} k={k} V={V} N={N} T={T}")
    from bcjr import bcjr_forward_backward
    seq, cb, g = _rng_case(L * 10 + N, 3, N, V, L)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, torch.tensor(cb, device="cuda"), T, L=L, k=k, V=V)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    for b in range(seq.shape[0]):
        bf = oracle.brute_force(seq[b], cb, T, L, k * V, g=g[b])
        assert max_rel(soft[b].detach().cpu().numpy(), bf["soft"]) < SOFT_TOL
        assert abs(float(logZ[b].detach()) - bf["logZ"]) <= LOGZ_TOL * max(1.0, abs(bf["logZ"]))
        assert max_rel(x.grad[b].cpu().numpy(), bf["grad"]) < GRAD_TOL


# (L, k, V, N, B, codebook kind, T)
CASES = [
    (12, 2, 1, 256, 8, "1mad", 0.1),     # CPU-runnable reference config (subset of B=128)
    (12, 2, 1, 256, 4, "1mad", 1.0),
    (12, 2, 1, 256, 4, "3inst", 0.3),
    (12, 2, 1, 256, 4, "table", 0.1),
    (13, 2, 1, 64, 3, "table", 0.2),
    (14, 2, 1, 64, 3, "3inst", 0.1),     # 2 butterflies per thread
    (15, 2, 1, 32, 2, "1mad", 0.1),      # 4 per thread
    (12, 2, 2, 128, 4, "table", 0.5),    # kV = 4 (reference QAT shape at L=12)
    (12, 2, 2, 128, 4, "hyb", 0.3),
    (10, 1, 1, 64, 4, "table", 0.2),     # kV = 1
    (10, 1, 2, 64, 4, "hyb", 0.4),       # k = 1, V = 2 (kV = 2, 2-D)
    (16, 2, 1, 256, 2, "3inst", 0.1),    # single-tile config: L=16, 8 butterflies per thread
    (16, 2, 1, 256, 2, "3inst", 1.0),    # its other two temperatures
    (16, 2, 1, 256, 2, "3inst", 0.3),
    (16, 2, 1, 96, 2, "1mad", 0.05),
    (16, 2, 1, 128, 2, "3inst", 0.01),   # the float32 floor the reference states (T >= 1e-2)
    (16, 2, 2, 64, 2, "hyb", 0.1),       # reference QAT trellis (L=16, kV=4)
    (16, 2, 1, 1024, 1, "3inst", 0.1),   # long sequence: per-step partials are double-buffered
    (16, 2, 1, 128, 2, "table", 0.2),    # table codebook on the 1024-thread forward
    (16, 2, 1, 64, 2, "1mad", 0.2),      # 1MAD group-sum variant: every alpha + mu butterfly cached
    (16, 1, 2, 64, 2, "hyb", 0.3),       # k = 1, V = 2 at L = 16: 8 two-dimensional butterflies per thread
    (16, 1, 2, 64, 2, "table", 0.15),
    (14, 2, 1, 64, 3, "1mad", 0.05),     # 1024-thread forward, group-sum variant below 0.08, 1 butterfly per thread
    (15, 2, 1, 64, 2, "3inst", 0.07),    # the same, 2 per thread
    (14, 2, 1, 64, 3, "1mad", 0.03),     # 1024-thread forward, exact variant, 1 butterfly per thread
    (15, 2, 1, 64, 2, "3inst", 0.04),    # 1024-thread forward, exact variant, 2 per thread
    (16, 2, 1, 64, 2, "3inst", 0.045),   # the 1024-thread forward's switch point
    (16, 2, 1, 64, 2, "3inst", 0.06),
    (15, 2, 1, 64, 2, "table", 0.3),
]


def _case_tensors(bcjr_mod, oracle, L, V, N, B, kind, seed):
    rng = np.random.default_rng(seed)
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    if kind == "table":
        cb_np = rng.standard_normal((1 << L, V)).astype(np.float32)
        cb = torch.tensor(cb_np, device="cuda")
    else:
        cb, cb_np = _codebook(bcjr_mod, oracle, kind, L, "cuda")
    return seq, g, cb, cb_np


@pytest.mark.parametrize("L,k,V,N,B,kind,T", CASES)
def test_forward_vs_oracle(bcjr_mod, oracle, L, k, V, N, B, kind, T):
    _say(f"forward L={L} k={k} V={V} N={N} B={B} {kind} T={T}")
    from bcjr import bcjr_forward_backward
    seq, g, cb, cb_np = _case_tensors(bcjr_mod, oracle, L, V, N, B, kind, seed=L + N + B)
    soft, logZ = bcjr_forward_backward(torch.tensor(seq, device="cuda"), cb, T, L=L, k=k, V=V)
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, T, L, k * V)
    assert max_rel(soft.cpu().numpy(), s_ref) < SOFT_TOL
    assert np.abs(logZ.cpu().numpy() - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()


@pytest.mark.parametrize("L,k,V,N,B,kind,T", CASES)
def test_backward_vs_oracle(bcjr_mod, oracle, L, k, V, N, B, kind, T):
    _say(f"backward L={L} k={k} V={V} N={N} B={B} {kind} T={T}")
    from bcjr import bcjr_forward_backward
    B = min(B, 3)
    seq, g, cb, cb_np = _case_tensors(bcjr_mod, oracle, L, V, N, B, kind, seed=3 * L + N)
    gz = np.random.default_rng(1).standard_normal(B).astype(np.float32)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, T, L=L, k=k, V=V)
    loss = (soft * torch.tensor(g, device="cuda")).sum() + (logZ * torch.tensor(gz, device="cuda")).sum()
    loss.backward()
    d_ref = oracle.bcjr_backward(seq, cb_np, T, L, k * V, g, gz)
    assert max_rel(x.grad.cpu().numpy(), d_ref) < GRAD_TOL


@pytest.mark.parametrize("Q,T", [(9, 1.0), (9, 0.03), (3, 0.2), (6, 0.1), (10, 0.1)])
def test_hyb_column_walk_vs_oracle(bcjr_mod, oracle, Q, T):
    """HYB at L=16, kV=4 runs the soft kernels on the column-walk LUT for
    3 <= Q <= 9 (Q = 10 keeps the signed LUT): forward and backward against the
    oracle on the materialised codebook, in the fast and the low-temperature
    (T < 0.08) variants."""
    _say(f"HYB column walk Q={Q} T={T}")
    from bcjr import bcjr_forward_backward
    L, k, V, N, B = 16, 2, 2, 32, 2
    rng = np.random.default_rng(100 + Q)
    lut = rng.standard_normal((1 << Q, 2)).astype(np.float32)
    cb = bcjr_mod.make_hyb_codebook_gpu(lut, Q=Q, L_bits=L, device="cuda")
    cb_np = cb.cpu().numpy()
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, T, L=L, k=k, V=V)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, T, L, k * V)
    assert max_rel(soft.detach().cpu().numpy(), s_ref) < SOFT_TOL
    assert np.abs(logZ.detach().cpu().numpy() - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()
    assert max_rel(x.grad.cpu().numpy(), oracle.bcjr_backward(seq, cb_np, T, L, k * V, g)) < GRAD_TOL


def test_hyb_column_walk_per_sequence_temperature(bcjr_mod, oracle):
    """One launch of the column-walk kernels whose sequences take both variants
    (T below and above 0.08) and the Viterbi over the same batch, against the
    oracle sequence by sequence."""
    _say("HYB column walk, per-sequence T")
    from bcjr import bcjr_forward_backward, viterbi_encode_v_batched_hip
    L, k, V, N = 16, 2, 2, 24
    Ts = np.array([0.05, 0.3, 0.02, 1.0], np.float32)
    B = len(Ts)
    rng = np.random.default_rng(31)
    cb, cb_np = _codebook(bcjr_mod, oracle, "hyb", L, "cuda")
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, torch.tensor(Ts, device="cuda"), L=L, k=k, V=V)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    for b in range(B):
        s_ref, z_ref = oracle.bcjr_forward(seq[b:b + 1], cb_np, float(Ts[b]), L, k * V)
        d_ref = oracle.bcjr_backward(seq[b:b + 1], cb_np, float(Ts[b]), L, k * V, g[b:b + 1])
        assert max_rel(soft[b:b + 1].detach().cpu().numpy(), s_ref) < SOFT_TOL
        assert max_rel(x.grad[b:b + 1].cpu().numpy(), d_ref) < GRAD_TOL
    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(torch.tensor(seq.reshape(B, N * V), device="cuda"),
                                                                cb, L=L, k=k, V=V, return_all=True)
    assert np.array_equal(out["walk"].cpu().numpy(), oracle.viterbi(seq, cb_np, L, k * V)[0])


@pytest.mark.parametrize("L,k,V,kind", [(12, 2, 1, "1mad"), (16, 2, 1, "3inst"), (16, 2, 2, "hyb")])
def test_short_and_empty_batches(bcjr_mod, oracle, L, k, V, kind):
    """Edge shapes: sequences of 1, 2 and 3 steps (forward, backward and Viterbi
    against the oracle) and an empty batch (empty outputs, zero-size gradient)."""
    _say(f"short/empty L={L} k={k} V={V} {kind}")
    from bcjr import bcjr_forward_backward, viterbi_encode_v_batched_hip
    cb, cb_np = _codebook(bcjr_mod, oracle, kind, L, "cuda")
    T = 0.2
    for N in (1, 2, 3):
        rng = np.random.default_rng(N)
        seq = rng.standard_normal((2, N, V)).astype(np.float32)
        g = rng.standard_normal((2, N, V)).astype(np.float32)
        x = torch.tensor(seq, device="cuda", requires_grad=True)
        soft, logZ = bcjr_forward_backward(x, cb, T, L=L, k=k, V=V)
        (soft * torch.tensor(g, device="cuda")).sum().backward()
        s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, T, L, k * V)
        assert max_rel(soft.detach().cpu().numpy(), s_ref) < SOFT_TOL
        assert np.abs(logZ.detach().cpu().numpy() - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()
        assert max_rel(x.grad.cpu().numpy(), oracle.bcjr_backward(seq, cb_np, T, L, k * V, g)) < GRAD_TOL
        bits, start, recon, mse, out = viterbi_encode_v_batched_hip(
            torch.tensor(seq.reshape(2, N * V), device="cuda"), cb, L=L, k=k, V=V, return_all=True)
        walk_r, _, start_r, recon_r, _ = oracle.viterbi(seq, cb_np, L, k * V)
        assert np.array_equal(out["walk"].cpu().numpy(), walk_r)
        assert np.array_equal(start.cpu().numpy(), start_r)
        assert np.array_equal(recon.cpu().numpy(), recon_r.reshape(2, N * V))
    x = torch.zeros((0, 8, V), device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, T, L=L, k=k, V=V)
    assert soft.shape == (0, 8, V) and logZ.shape == (0,)
    soft.sum().backward()
    assert x.grad.shape == (0, 8, V)
    bits, start, recon, mse = viterbi_encode_v_batched_hip(torch.zeros((0, 8 * V), device="cuda"), cb,
                                                           L=L, k=k, V=V)
    assert bits.shape[0] == 0 and start.shape == (0,) and recon.shape == (0, 8 * V)


def test_longest_sequences_and_lds_limit(bcjr_mod, oracle):
    """Maximum sizes at L=16, V=1 (3INST, T=0.1): the backward's longest
    sequence (N = 2024) and the forward's (N = 2704: the 1024-thread forward
    holds N <= 2702, so 2703 and 2704 take the 512-thread forward) against the
    oracle, and one step more is refused (BcjrError naming the LDS need) before
    any launch."""
    _say("longest sequences L=16")
    from bcjr import bcjr_forward_backward, make_3inst_codebook
    from bcjr import ops
    from bcjr._lib import BcjrError
    L = 16
    cb = make_3inst_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    spec, _ = bcjr_mod.codes.resolve_codebook(cb, L, 2, 1, torch.device("cuda"))
    rng = np.random.default_rng(11)
    seq = rng.standard_normal((1, 2024, 1)).astype(np.float32)
    g = rng.standard_normal((1, 2024, 1)).astype(np.float32)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, 0.1, L=L, k=2, V=1)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, 0.1, L, 2)
    assert max_rel(soft.detach().cpu().numpy(), s_ref) < SOFT_TOL
    assert max_rel(x.grad.cpu().numpy(), oracle.bcjr_backward(seq, cb_np, 0.1, L, 2, g)) < GRAD_TOL
    for n in (2702, 2704):
        seq2 = rng.standard_normal((1, n, 1)).astype(np.float32)
        soft2, _ = ops.forward(spec, torch.tensor(seq2, device="cuda"), 0.1, None)
        assert max_rel(soft2.cpu().numpy(), oracle.bcjr_forward(seq2, cb_np, 0.1, L, 2)[0]) < SOFT_TOL, n
    with pytest.raises(BcjrError, match="LDS"):
        ops.forward(spec, torch.zeros((1, 2705, 1), device="cuda"), 0.1, None)
    with pytest.raises(BcjrError, match="LDS"):
        ops.backward(spec, torch.zeros((1, 2025, 1), device="cuda"), 0.1, None, torch.zeros((1, 2025, 1), device="cuda"))


@pytest.mark.parametrize("T", [0.03, 0.045, 0.05, 0.07, 0.08, 0.1])
def test_heavy_tailed_weights_near_the_variant_switch_points(bcjr_mod, oracle, T):
    """L=16 layer instances (1024-thread forward, 8-butterfly backward) on
    Student-t (3 degrees of freedom) weights clipped at |w| <= 6 -- tails up to
    twice the codebook's range (|c| < 3.2) -- at temperatures on both sides of
    the forward's (0.045) and the backward's (0.08) switch from the group-sum to
    the exact-maximum variant, where the group-sum variant meets groups near its
    recompute threshold.  The bars of the Gaussian configs hold."""
    _say(f"student-t weights L=16 T={T}")
    from bcjr import bcjr_forward_backward, make_3inst_codebook
    L, N, B = 16, 256, 3
    rng = np.random.default_rng(int(T * 1000))
    seq = np.clip(rng.standard_t(3, size=(B, N, 1)), -6.0, 6.0).astype(np.float32)
    g = rng.standard_normal((B, N, 1)).astype(np.float32)
    cb = make_3inst_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, T, L=L, k=2, V=1)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, T, L, 2)
    d_ref = oracle.bcjr_backward(seq, cb_np, T, L, 2, g)
    assert max_rel(soft.detach().cpu().numpy(), s_ref) < SOFT_TOL
    assert np.abs(logZ.detach().cpu().numpy() - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()
    assert max_rel(x.grad.cpu().numpy(), d_ref) < GRAD_TOL


def test_extreme_outliers_against_the_reference_float32_order(bcjr_mod, oracle):
    """Unclipped Student-t (3) weights (|w| up to ~17, five times the codebook's
    range) at T=0.05: log-domain values reach ~-10^4 there and float32 cannot
    hold them to 1e-4 -- the reference's own eager algorithm in float32
    (expansion-form emission, gather + logsumexp: oracle/torch_ref.py) is off by
    ~2e-3 on this input.  The kernel must stay at least four times closer to the
    float64 oracle than that, with log Z at its usual bar."""
    _say("extreme outliers vs the float32 reference order")
    from bcjr import bcjr_forward_backward, make_3inst_codebook
    from oracle.torch_ref import eager_bcjr
    L, T = 16, 0.05
    rng = np.random.default_rng(50)
    seq = rng.standard_t(3, size=(3, 256, 1)).astype(np.float32)
    cb = make_3inst_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    soft, logZ = bcjr_forward_backward(torch.tensor(seq, device="cuda"), cb, T, L=L, k=2, V=1)
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, T, L, 2)
    with torch.no_grad():
        s32, _ = eager_bcjr(torch.tensor(seq), torch.tensor(cb_np), T, L, 2, checkpoint=False)
    ref_err = max_rel(s32.numpy(), s_ref)
    err = max_rel(soft.cpu().numpy(), s_ref)
    assert ref_err > SOFT_TOL  # the input is beyond float32's reach, as intended
    assert err < ref_err / 4, (err, ref_err)
    assert np.abs(logZ.cpu().numpy() - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()


def test_per_sequence_temperature(bcjr_mod, oracle):
    _say("per-sequence T")
    from bcjr import bcjr_forward_backward
    L, N, B = 12, 64, 6
    seq, g, cb, cb_np = _case_tensors(bcjr_mod, oracle, L, 1, N, B, "3inst", seed=4)
    Ts = np.array([0.05, 0.08, 0.12, 0.2, 0.3, 0.5], np.float32)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, torch.tensor(Ts, device="cuda"), L=L, k=2, V=1)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    for b in range(B):
        s_ref, z_ref = oracle.bcjr_forward(seq[b:b + 1], cb_np, float(Ts[b]), L, 2)
        d_ref = oracle.bcjr_backward(seq[b:b + 1], cb_np, float(Ts[b]), L, 2, g[b:b + 1])
        assert max_rel(soft[b:b + 1].detach().cpu().numpy(), s_ref) < SOFT_TOL
        assert max_rel(x.grad[b:b + 1].cpu().numpy(), d_ref) < GRAD_TOL


def test_return_internals_vs_gather_form(bcjr_mod, oracle):
    _say("return_internals")
    from bcjr import bcjr_forward_backward
    L, k, V, N, T = 8, 2, 1, 12, 0.3
    seq, cb, _ = _rng_case(21, 2, N, V, L)
    soft, logZ, P, la, lb = bcjr_forward_backward(torch.tensor(seq, device="cuda"),
                                                  torch.tensor(cb, device="cuda"), T,
                                                  L=L, k=k, V=V, return_internals=True)
    s2, z2, P2, la2, lb2 = oracle.naive_forward(seq, cb, T, L, k * V, return_internals=True)
    assert max_rel(soft.cpu().numpy(), s2) < SOFT_TOL
    assert np.abs(P.cpu().numpy() - P2).max() < 1e-5
    assert np.abs(la.cpu().numpy() - la2).max() < 1e-4 * np.abs(la2).max()
    assert np.abs(lb.cpu().numpy() - lb2).max() < 1e-4 * max(1.0, np.abs(lb2).max())


def test_monolithic_wrapper_and_dtype(bcjr_mod, oracle):
    _say("monolithic wrapper")
    from bcjr import bcjr_forward_backward_monolithic
    L, k, V, N, T = 12, 2, 2, 32, 1.0
    seq, cb, g = _rng_case(8, 2, N, V, L)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, none = bcjr_forward_backward_monolithic(x, torch.tensor(cb, device="cuda"),
                                                  torch.tensor(T, device="cuda"), L=L, k=k, V=V)
    assert none is None and soft.dtype == torch.float32
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    assert max_rel(soft.detach().cpu().numpy(), oracle.bcjr_forward(seq, cb, T, L, 4)[0]) < SOFT_TOL
    assert max_rel(x.grad.cpu().numpy(), oracle.bcjr_backward(seq, cb, T, L, 4, g)) < GRAD_TOL


@pytest.mark.parametrize("B,N,loss", [(2, 8, "randn"), (4, 16, "sum")])
def test_reference_node_gates_l16_kv4(bcjr_mod, oracle, B, N, loss):
    """The shapes of the reference's own node gates at the module defaults (L=16,
    k=2, V=2): B=2, N=8 with a random upstream gradient
    (test_bcjr_monolithic_parity.py:23-53) and B=4, N=16 with loss soft.sum()
    (test_bcjr_fast_parity.py:23-57); codebook randn(2^16, 2), T = 1.0 as a 0-d
    device tensor, preds/succs passed as the callers pass them."""
    _say(f"reference node gate B={B} N={N} loss={loss}")
    from bcjr import bcjr_forward_backward, build_pred_succ_tables
    L, k, V, T = 16, 2, 2, 1.0
    rng = np.random.default_rng(100 + B)
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    g = (rng.standard_normal((B, N, V)) if loss == "randn" else np.ones((B, N, V))).astype(np.float32)
    preds, succs = build_pred_succ_tables(device="cuda")
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, torch.tensor(cb, device="cuda"), torch.tensor(T, device="cuda"),
                                       preds=preds, succs=succs)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    s_ref, z_ref = oracle.bcjr_forward(seq, cb, T, L, k * V)
    assert max_rel(soft.detach().cpu().numpy(), s_ref) < SOFT_TOL
    assert np.abs(logZ.detach().cpu().numpy() - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()
    assert max_rel(x.grad.cpu().numpy(), oracle.bcjr_backward(seq, cb, T, L, k * V, g)) < GRAD_TOL


def test_reference_variant_entry_points_are_the_node(bcjr_mod):
    """The reference's alternative implementations (forward_backward_fast.py:75,
    bcjr_graph.py:56, bcjr_monolithic_graph.py:41, bcjr_quant.py:63) are gated
    against its eager node at 1e-3 (test_bcjr_{fast,graph,mono_graph}_parity.py);
    here each is the same node, so values and gradients are identical."""
    _say("variant entry points")
    from bcjr.quant import _bcjr_chunk_forward
    L, k, V, B, N = 12, 2, 2, 4, 16
    rng = np.random.default_rng(7)
    cb = torch.tensor(rng.standard_normal((1 << L, V)).astype(np.float32), device="cuda")
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    T = torch.tensor(1.0, device="cuda")
    outs, grads = [], []
    fns = [lambda x: bcjr_mod.bcjr_forward_backward(x, cb, T, L=L, k=k, V=V)[0],
           lambda x: bcjr_mod.bcjr_forward_backward_fast(x, cb, T, L=L, k=k, V=V)[0],
           lambda x: bcjr_mod.bcjr_forward_backward_monolithic_graphed(x, cb, T, L=L, k=k, V=V)[0]]
    for fn in fns:
        x = torch.tensor(seq, device="cuda", requires_grad=True)
        soft = fn(x)
        soft.sum().backward()
        outs.append(soft.detach())
        grads.append(x.grad)
    for o, g in zip(outs[1:], grads[1:]):
        assert torch.equal(o, outs[0]) and torch.equal(g, grads[0])
    # the chunk forwards use the module defaults L=16, k=2, V=2, as in the reference
    lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
    cb16 = bcjr_mod.make_hyb_codebook_gpu(lut, 9, 16, "cuda")
    x = torch.tensor(rng.standard_normal((2, 32, 2)).astype(np.float32), device="cuda")
    ref = bcjr_mod.bcjr_forward_backward(x, cb16, T)[0]
    assert torch.equal(bcjr_mod.graphed_bcjr_chunk_forward(x, cb16, T, None, None), ref)
    assert torch.equal(_bcjr_chunk_forward(x, cb16, T), ref)
    bcjr_mod.reset_graph_cache()
    bcjr_mod.reset_mono_graph_cache()


def test_toy_two_layer_gradients_reach_every_latent(bcjr_mod):
    """Integration gate in the manner of test_llama_bcjr_toy.py:37-157 (every
    W_latent gets a non-zero gradient): a two-layer MLP whose weights are soft-
    quantized by bcjr_quantize_weight (RHT, BCJR at L=16 kV=4 HYB, inverse RHT),
    one loss, one backward."""
    _say("toy two-layer gradients")
    lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr_mod.make_hyb_codebook_gpu(lut, 9, 16, "cuda")
    torch.manual_seed(0)
    shapes = [(64, 32), (16, 64)]
    latents = [(torch.randn(s, device="cuda") * 0.05).requires_grad_(True) for s in shapes]
    signs = [(torch.tensor(bcjr_mod.make_sign_vector(s[0], 2 * i), device="cuda"),
              torch.tensor(bcjr_mod.make_sign_vector(s[1], 2 * i + 1), device="cuda")) for i, s in enumerate(shapes)]
    T = torch.tensor(0.3, device="cuda")
    x = torch.randn(8, 32, device="cuda")
    h = x
    for W, (sl, sr) in zip(latents, signs):
        Wq = bcjr_mod.bcjr_quantize_weight(W, sl, sr, cb, T)
        assert Wq.shape == W.shape and torch.isfinite(Wq).all()
        h = torch.nn.functional.gelu(h @ Wq.t())
    loss = (h - torch.randn_like(h)).pow(2).mean()
    loss.backward()
    for W in latents:
        assert W.grad is not None and torch.isfinite(W.grad).all()
        assert (W.grad != 0).any() and W.grad.abs().max() > 0


def test_quantize_weight_rotated(bcjr_mod, oracle):
    """Tile -> node -> untile around the RMS scale (bcjr_quant.py:125-156)."""
    _say("quantize_weight_rotated")
    from bcjr import bcjr_quantize_weight_rotated
    from bcjr.quant import tile_for_viterbi
    L = 12
    cb, cb_np = _codebook(bcjr_mod, oracle, "1mad", L, "cuda")
    W = torch.randn(64, 32, device="cuda", generator=torch.Generator("cuda").manual_seed(0)) * 0.02
    W.requires_grad_(True)
    Wq = bcjr_quantize_weight_rotated(W, cb, 0.1, L=L, k=2, V=1)
    g = torch.randn_like(Wq)
    (Wq * g).sum().backward()
    scale = W.detach().pow(2).mean().sqrt()
    seqs, info = tile_for_viterbi((W.detach() / scale))
    s_ref, _ = oracle.bcjr_forward(seqs.cpu().numpy()[:, :, None], cb_np, 0.1, L, 2)
    ref = torch.tensor(s_ref[:, :, 0]).reshape(info[1], 64, 16).permute(1, 0, 2).reshape(64, 32) * scale.cpu()
    assert max_rel(Wq.detach().cpu().numpy(), ref.numpy()) < SOFT_TOL
    gseq, _ = tile_for_viterbi(g.detach())
    d_ref = oracle.bcjr_backward(seqs.cpu().numpy()[:, :, None], cb_np, 0.1, L, 2, gseq.cpu().numpy()[:, :, None])
    d_ref = torch.tensor(d_ref[:, :, 0]).reshape(info[1], 64, 16).permute(1, 0, 2).reshape(64, 32)
    assert max_rel(W.grad.cpu().numpy(), d_ref.numpy()) < GRAD_TOL


# --------------------------------------------------------------------------
# Viterbi (T -> 0): bit-exact
# --------------------------------------------------------------------------

def test_viterbi_toy_known_answer(bcjr_mod):
    _say("viterbi toy")
    from bcjr import viterbi_encode_v_batched_hip
    cb = torch.tensor([[-1.2], [-0.3], [0.4], [1.1]], device="cuda")
    seq = torch.tensor([[-1.0, 0.5, 0.8]], device="cuda")
    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(seq, cb, L=2, k=1, V=1, return_all=True)
    assert recon.cpu().numpy().ravel().tolist() == pytest.approx([-1.2, -0.3, 1.1], abs=1e-6)
    assert abs(float(((recon - seq) ** 2).sum()) - 0.77) < 1e-4
    assert out["walk"].cpu().tolist() == [[0, 1, 3]] and int(start[0]) == 0


VIT_CASES = [  # (L, k, V, N, B, kind)
    (12, 2, 1, 256, 8, "1mad"),
    (12, 2, 1, 256, 8, "3inst"),
    (12, 2, 1, 100, 5, "table"),
    (12, 2, 2, 128, 4, "hyb"),
    (12, 2, 2, 128, 4, "table"),
    (10, 1, 1, 64, 4, "table"),
    (10, 1, 2, 64, 4, "hyb"),
    (16, 2, 1, 256, 4, "1mad"),
    (16, 2, 1, 256, 4, "3inst"),
    (16, 2, 2, 128, 2, "hyb"),         # 1024 threads, 16 interleaved LUT copies
    (15, 1, 2, 64, 2, "hyb"),          # 1024 threads, cached codewords, 2 butterflies per thread
    (14, 2, 1, 128, 3, "3inst"),       # 1024 threads, one butterfly per thread
    (16, 1, 2, 64, 2, "table"),        # 1024 threads, 4 uncached butterflies per thread
    (16, 1, 2, 64, 2, "hyb"),          # 512 threads, one LUT copy (the copies do not fit beside 2^14 states)
]


@pytest.mark.parametrize("L,k,V,N,B,kind", VIT_CASES)
def test_viterbi_bit_exact(bcjr_mod, oracle, L, k, V, N, B, kind):
    _say(f"viterbi L={L} k={k} V={V} N={N} B={B} {kind}")
    from bcjr import viterbi_decode_v_batched, viterbi_encode_v_batched_hip
    seq, _, cb, cb_np = _case_tensors(bcjr_mod, oracle, L, V, N, B, kind, seed=L * 7 + N)
    x = torch.tensor(seq.reshape(B, N * V), device="cuda")
    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(x, cb, L=L, k=k, V=V, return_all=True)
    walk_r, bits_r, start_r, recon_r, mse_r = oracle.viterbi(seq, cb_np, L, k * V)
    assert (out["walk"].cpu().numpy() == walk_r).all()
    assert (bits.cpu().numpy() == bits_r).all()
    assert (start.cpu().numpy() == start_r).all()
    assert (recon.cpu().numpy() == recon_r.reshape(B, N * V)).all()
    assert np.abs(mse.cpu().numpy() - mse_r).max() < 1e-6
    if out["packed"] is not None:
        assert (out["packed"].cpu().numpy() == oracle.pack_bits(bits_r, k * V)).all()
        w2, r2 = viterbi_decode_v_batched(None, start, cb, L=L, k=k, V=V, packed=out["packed"], N=N)
        assert (w2.cpu().numpy() == walk_r).all()
    w3, r3 = viterbi_decode_v_batched(bits, start, cb, L=L, k=k, V=V)
    assert (w3.cpu().numpy() == walk_r).all() and (r3.cpu().numpy() == recon_r.reshape(B, -1)).all()


@pytest.mark.parametrize("Q", [3, 6, 9, 10])
def test_viterbi_hyb_column_walk(bcjr_mod, oracle, Q):
    """The 1024-thread Viterbi at L=16, kV=4 reads the column-walk LUT for
    3 <= Q <= 9 (Q = 10: the signed LUT copies): bit-exact against the oracle."""
    _say(f"viterbi HYB column walk Q={Q}")
    from bcjr import viterbi_encode_v_batched_hip
    L, k, V, N, B = 16, 2, 2, 48, 3
    rng = np.random.default_rng(200 + Q)
    lut = rng.standard_normal((1 << Q, 2)).astype(np.float32)
    cb = bcjr_mod.make_hyb_codebook_gpu(lut, Q=Q, L_bits=L, device="cuda")
    cb_np = cb.cpu().numpy()
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(torch.tensor(seq.reshape(B, N * V), device="cuda"),
                                                                cb, L=L, k=k, V=V, return_all=True)
    walk_r, bits_r, start_r, recon_r, mse_r = oracle.viterbi(seq, cb_np, L, k * V)
    assert np.array_equal(out["walk"].cpu().numpy(), walk_r)
    assert np.array_equal(start.cpu().numpy(), start_r)
    assert np.array_equal(recon.cpu().numpy(), recon_r.reshape(B, N * V))


def test_viterbi_tie_rules(bcjr_mod, oracle):
    _say("viterbi ties")
    from bcjr import viterbi_encode_v_batched_hip
    L, N = 8, 6
    cb = np.zeros((1 << L, 1), np.float32)
    cb[5] = cb[77] = 0.5
    seq = np.full((2, N), 0.5, np.float32)
    seq[1, :3] = 0.0
    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(
        torch.tensor(seq, device="cuda"), torch.tensor(cb, device="cuda"), L=L, k=2, V=1, return_all=True)
    walk_r, bits_r, start_r, _, _ = oracle.viterbi(seq[:, :, None], cb, L, 2)
    assert (out["walk"].cpu().numpy() == walk_r).all() and (start.cpu().numpy() == start_r).all()


def test_viterbi_table1_band_l16(bcjr_mod):
    """Table-1 distortion band at L=16, k=2 (src/tripwires/test_viterbi.py:77-133)."""
    _say("viterbi table-1 band")
    from bcjr import make_1mad_codebook, make_3inst_codebook, viterbi_encode_v_batched_hip
    seq = torch.tensor(np.random.default_rng(42).standard_normal((64, 256)).astype(np.float32), device="cuda")
    for make in (make_1mad_codebook, make_3inst_codebook):
        _, _, _, mse = viterbi_encode_v_batched_hip(seq, make(16, "cuda"), L=16, k=2, V=1)
        assert 0.062 <= float(mse.mean()) <= 0.075


# --------------------------------------------------------------------------
# full-size properties (single-tile config: L=16, k=2, V=1, N=256)
# --------------------------------------------------------------------------

def test_full_size_properties(bcjr_mod):
    _say("full-size properties B=512")
    from bcjr import bcjr_forward_backward, make_3inst_codebook, viterbi_encode_v_batched_hip
    torch.manual_seed(0)
    B, N = 512, 256
    cb = make_3inst_codebook(16, "cuda")
    x = torch.randn(B, N, 1, device="cuda")
    soft, logZ = bcjr_forward_backward(x, cb, 0.1, L=16, k=2, V=1)
    assert torch.isfinite(soft).all() and torch.isfinite(logZ).all()
    assert float(soft.min()) >= float(cb.min()) - 1e-5 and float(soft.max()) <= float(cb.max()) + 1e-5
    # order independence: a permuted batch gives the permuted results
    perm = torch.randperm(B, device="cuda")
    soft_p, _ = bcjr_forward_backward(x[perm], cb, 0.1, L=16, k=2, V=1)
    assert torch.equal(soft_p, soft[perm])
    # the backward is linear in the upstream gradient
    xs = x[:64].clone().requires_grad_(True)
    g1, g2 = torch.randn_like(xs), torch.randn_like(xs)
    grads = []
    for g in (g1, g2, g1 + g2):
        xs.grad = None
        s, _ = bcjr_forward_backward(xs, cb, 0.1, L=16, k=2, V=1)
        (s * g).sum().backward()
        grads.append(xs.grad.clone())
    assert max_rel((grads[0] + grads[1]).cpu().numpy(), grads[2].cpu().numpy()) < 1e-4
    # T -> 0 approaches the Viterbi reconstruction wherever the best path is not
    # tied to within ~T (at T=1e-3 about 0.3-1.2% of positions still mix, in the
    # float64 oracle too)
    s_lo, _ = bcjr_forward_backward(x[:64], cb, 1e-3, L=16, k=2, V=1)
    _, _, recon, _ = viterbi_encode_v_batched_hip(x[:64, :, 0].contiguous(), cb, L=16, k=2, V=1)
    diff = (s_lo[:, :, 0] - recon).abs()
    assert float((diff > 1e-2).float().mean()) < 0.05
    assert float(diff.median()) < 1e-4


def test_cpu_config_every_sequence_vs_oracle(bcjr_mod, oracle):
    """The CPU-runnable config whole: L=12 (4,096 states), k=2, V=1, N=256, all
    128 sequences of N(0,1) weights (seed 0), 1MAD, T=0.1, upstream gradient
    N(0,1) (seed 1): soft, log Z and the gradient of every sequence against the
    oracle, and the Viterbi path of every sequence bit-exact."""
    _say("cpu config: all 128 sequences")
    from bcjr import bcjr_forward_backward, make_1mad_codebook, viterbi_encode_v_batched_hip
    B, N, L = 128, 256, 12
    seq = np.random.default_rng(0).standard_normal((B, N, 1)).astype(np.float32)
    g = np.random.default_rng(1).standard_normal((B, N, 1)).astype(np.float32)
    cb = make_1mad_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, 0.1, L=L, k=2, V=1)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, 0.1, L, 2)
    d_ref = oracle.bcjr_backward(seq, cb_np, 0.1, L, 2, g)
    soft_h, z_h, d_h = soft.detach().cpu().numpy(), logZ.detach().cpu().numpy(), x.grad.cpu().numpy()
    for b in range(B):  # the bars hold per sequence, not only over the batch
        assert max_rel(soft_h[b], s_ref[b]) < SOFT_TOL, f"seq {b}: soft"
        assert abs(float(z_h[b]) - float(z_ref[b])) <= LOGZ_TOL * abs(float(z_ref[b])), f"seq {b}: logZ"
        assert max_rel(d_h[b], d_ref[b]) < GRAD_TOL, f"seq {b}: grad"
    bits, start, recon, _, out = viterbi_encode_v_batched_hip(x.detach()[:, :, 0].contiguous(), cb, L=L, k=2, V=1,
                                                              return_all=True)
    walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(seq, cb_np, L, 2)
    assert (out["walk"].cpu().numpy() == walk_r).all()
    assert (bits.cpu().numpy() == bits_r).all() and (start.cpu().numpy() == start_r).all()
    assert (recon.cpu().numpy() == recon_r.reshape(B, N)).all()


@pytest.mark.parametrize("T", [0.1, 1.0, 0.3])
def test_bench_batch_spot_check_vs_oracle(bcjr_mod, oracle, T):
    """The single-tile workload at its full size (B=4096: each workgroup reuses its
    HBM slot for ~16 sequences) at each of its temperatures: eight sequences of
    the batch (both ends, the middle and the slot-reuse boundaries around it)
    against the oracle -- soft, log Z and gradient -- and, at T=0.1, the Viterbi
    path bit-exact."""
    _say(f"bench batch spot check B=4096 T={T}")
    from bcjr import bcjr_forward_backward, make_3inst_codebook, viterbi_encode_v_batched_hip
    B, N, L = 4096, 256, 16
    rng = np.random.default_rng(0)
    seq = rng.standard_normal((B, N, 1)).astype(np.float32)
    g = rng.standard_normal((B, N, 1)).astype(np.float32)
    cb = make_3inst_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, T, L=L, k=2, V=1)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    assert torch.isfinite(soft).all() and torch.isfinite(x.grad).all()
    pick = [0, 1, 255, 256, 2047, 2048, 4094, 4095]
    s_ref, z_ref = oracle.bcjr_forward(seq[pick], cb_np, T, L, 2)
    d_ref = oracle.bcjr_backward(seq[pick], cb_np, T, L, 2, g[pick])
    assert max_rel(soft.detach().cpu().numpy()[pick], s_ref) < SOFT_TOL
    assert np.abs(logZ.detach().cpu().numpy()[pick] - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()
    assert max_rel(x.grad.cpu().numpy()[pick], d_ref) < GRAD_TOL
    if T != 0.1:
        return
    bits, start, recon, _, out = viterbi_encode_v_batched_hip(x.detach()[:, :, 0].contiguous(), cb, L=L, k=2, V=1,
                                                              return_all=True)
    walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(seq[pick], cb_np, L, 2)
    assert (out["walk"].cpu().numpy()[pick] == walk_r).all()
    assert (bits.cpu().numpy()[pick] == bits_r).all() and (start.cpu().numpy()[pick] == start_r).all()
    assert (recon.cpu().numpy()[pick] == recon_r.reshape(len(pick), N)).all()


def test_qat_shape_batch_spot_check_vs_oracle(bcjr_mod, oracle):
    """The reference's QAT shape at the bench's size (L=16, k=2, V=2, HYB Q=9,
    N=128, B=4096: the column-walk kernels, each workgroup reusing its slot for
    ~5 sequences): four sequences against the oracle -- soft, log Z and gradient
    at T=0.1, and the Viterbi path bit-exact."""
    _say("QAT shape batch spot check B=4096")
    from bcjr import bcjr_forward_backward, viterbi_encode_v_batched_hip
    B, N, L, V = 4096, 128, 16, 2
    rng = np.random.default_rng(3)
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    cb, cb_np = _codebook(bcjr_mod, oracle, "hyb", L, "cuda")
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, 0.1, L=L, k=2, V=V)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    bits, start, recon, _, out = viterbi_encode_v_batched_hip(x.detach().reshape(B, N * V), cb, L=L, k=2, V=V,
                                                              return_all=True)
    pick = [0, 1, 2047, 4095]
    s_ref, z_ref = oracle.bcjr_forward(seq[pick], cb_np, 0.1, L, 4)
    d_ref = oracle.bcjr_backward(seq[pick], cb_np, 0.1, L, 4, g[pick])
    assert max_rel(soft.detach().cpu().numpy()[pick], s_ref) < SOFT_TOL
    assert np.abs(logZ.detach().cpu().numpy()[pick] - z_ref).max() <= LOGZ_TOL * np.abs(z_ref).max()
    assert max_rel(x.grad.cpu().numpy()[pick], d_ref) < GRAD_TOL
    walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(seq[pick], cb_np, L, 4)
    assert (out["walk"].cpu().numpy()[pick] == walk_r).all()
    assert (bits.cpu().numpy()[pick] == bits_r).all() and (start.cpu().numpy()[pick] == start_r).all()
    assert (recon.cpu().numpy()[pick] == recon_r.reshape(len(pick), N * V)).all()


def test_column_walk_many_sequences_per_workgroup_mixed_variants(bcjr_mod, oracle):
    """The column-walk kernels keep per-step tables, the codeword bases and (in
    the forward) codeword copies in LDS and registers from one sequence to the
    next of a workgroup.  B = 2048 sequences (about three per resident
    workgroup) whose T cycles through the group-sum and the exact variants, one
    with a NaN weight in the middle: late sequences against the oracle (soft,
    log Z, gradient, Viterbi walk), the NaN one NaN."""
    _say("column walk, B=2048 mixed T")
    from bcjr import bcjr_forward_backward, viterbi_encode_v_batched_hip
    B, N, L, V = 2048, 128, 16, 2
    rng = np.random.default_rng(17)
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    Ts = np.resize(np.array([0.05, 0.3, 1.0, 0.02, 0.1], np.float32), B)
    bad = 1027
    seq[bad, 5, 1] = np.nan
    cb, cb_np = _codebook(bcjr_mod, oracle, "hyb", L, "cuda")
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, torch.tensor(Ts, device="cuda"), L=L, k=2, V=V)
    (torch.nan_to_num(soft) * torch.tensor(g, device="cuda")).sum().backward()
    assert torch.isnan(soft[bad]).all() and torch.isnan(x.grad[bad]).all()
    for b in (1026, 1028, 1790, 2045, 2046, 2047):
        s_ref, z_ref = oracle.bcjr_forward(seq[b:b + 1], cb_np, float(Ts[b]), L, 4)
        d_ref = oracle.bcjr_backward(seq[b:b + 1], cb_np, float(Ts[b]), L, 4, g[b:b + 1])
        assert max_rel(soft[b:b + 1].detach().cpu().numpy(), s_ref) < SOFT_TOL, b
        assert abs(float(logZ[b].detach()) - float(z_ref[0])) <= LOGZ_TOL * abs(float(z_ref[0])), b
        assert max_rel(x.grad[b:b + 1].cpu().numpy(), d_ref) < GRAD_TOL, b
    good = np.array([1790, 2045, 2046, 2047])
    _, _, _, _, out = viterbi_encode_v_batched_hip(torch.tensor(seq.reshape(B, N * V), device="cuda"), cb,
                                                   L=L, k=2, V=V, return_all=True)
    walk_r = oracle.viterbi(seq[good], cb_np, L, 4)[0]
    assert np.array_equal(out["walk"].cpu().numpy()[good], walk_r)


def test_low_temperature_precision_bound(bcjr_mod, oracle):
    """Below T = 1e-2 float32 log-domain recursions lose precision as 1/T (the
    alpha/beta of a state on the final best path can lie ~1e4/T log2-units below
    the per-step maximum).  Record the bound: 2e-3 at T = 1e-3 (1e-4 holds for
    T >= 1e-2, see the parity cases)."""
    _say("low-T precision bound")
    from bcjr import bcjr_forward_backward, make_3inst_codebook
    cb = make_3inst_codebook(16, "cuda")
    x = np.random.default_rng(0).standard_normal((4, 256, 1)).astype(np.float32)
    soft, _ = bcjr_forward_backward(torch.tensor(x, device="cuda"), cb, 1e-3, L=16, k=2, V=1)
    s_ref, _ = oracle.bcjr_forward(x, cb.cpu().numpy(), 1e-3, 16, 2)
    assert max_rel(soft.cpu().numpy(), s_ref) < 2e-3


def test_graph_capture_replays(bcjr_mod):
    """Forward + backward captured in a HIP graph replay to the eager result."""
    _say("graph capture")
    from bcjr import bcjr_forward_backward, make_1mad_codebook
    L, B, N = 12, 16, 256
    cb = make_1mad_codebook(L, "cuda")
    T = torch.tensor(0.1, device="cuda")  # a 0-d device buffer, as QuantizedLinear.T_temp
    x = torch.randn(B, N, 1, device="cuda", requires_grad=True)
    g = torch.randn(B, N, 1, device="cuda")
    soft, _ = bcjr_forward_backward(x, cb, T, L=L, k=2, V=1)
    soft.backward(g)
    ref_soft, ref_grad = soft.detach().clone(), x.grad.clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        xg = x.detach().clone().requires_grad_(True)  # fresh leaf: its grad node lives on s
        for _ in range(2):  # warm the allocator and the launch-plan cache outside the capture
            xg.grad = None
            out, _ = bcjr_forward_backward(xg, cb, T, L=L, k=2, V=1)
            out.backward(g)
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    xg.grad = None
    with torch.cuda.graph(graph):
        out, _ = bcjr_forward_backward(xg, cb, T, L=L, k=2, V=1)
        out.backward(g)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.detach(), ref_soft)
        assert torch.equal(xg.grad, ref_grad)
        _ = torch.randn(1024, device="cuda").sum().item()  # eager work between replays
