"""CPU tests that pin the oracle (oracle/bcjr_oracle.c + oracle/__init__.py).

Each check is independent of the recursion it tests: exhaustive path
enumeration, finite differences, closed-form limits, the reference's own known
answers (src/tripwires/test_viterbi.py:17-53, Table-1 bands :77-133, codebook
bands src/tripwires/test_codes.py:27-98) and golden vectors produced by the
reference generators (tests/golden/code_vectors.json).
"""
import hashlib
import json
import os

import numpy as np
import pytest
from scipy import stats

from conftest import max_rel

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "code_vectors.json")

# (L, kV, V, N, T): tiny trellises brute force can enumerate.
TINY = [
    (4, 2, 1, 5, 0.7),
    (4, 2, 2, 4, 1.3),
    (6, 2, 1, 5, 0.3),
    (4, 1, 1, 6, 0.5),
    (3, 1, 1, 5, 0.2),
    (8, 4, 2, 3, 1.0),
    (6, 2, 1, 4, 0.05),
]


@pytest.mark.parametrize("L,KV,V,N,T", TINY)
def test_forward_matches_brute_force(oracle, L, KV, V, N, T):
    rng = np.random.default_rng(L * 100 + N)
    B = 3
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    soft, logZ = oracle.bcjr_forward(seq, cb, T, L, KV)
    for b in range(B):
        bf = oracle.brute_force(seq[b], cb, T, L, KV)
        assert np.abs(bf["soft"] - soft[b]).max() < 2e-6
        assert abs(bf["logZ"] - logZ[b]) < 2e-5 * max(1.0, abs(bf["logZ"]))


@pytest.mark.parametrize("L,KV,V,N,T", TINY)
def test_backward_matches_brute_force(oracle, L, KV, V, N, T):
    rng = np.random.default_rng(7 + L * 100 + N)
    B = 2
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    g = rng.standard_normal((B, N, V)).astype(np.float32)
    gz = rng.standard_normal(B).astype(np.float32)
    d = oracle.bcjr_backward(seq, cb, T, L, KV, g, gz)
    for b in range(B):
        bf = oracle.brute_force(seq[b], cb, T, L, KV, g=g[b], g_logZ=float(gz[b]))
        assert max_rel(d[b], bf["grad"]) < 1e-6


@pytest.mark.parametrize("L,KV,V,N,T", [c for c in TINY if (1 << c[0]) * (1 << c[1]) ** (c[3] - 1) <= 20000][:3])
def test_brute_force_gradient_is_the_derivative(oracle, L, KV, V, N, T):
    """The covariance closed form equals central differences of the enumerated loss."""
    rng = np.random.default_rng(3)
    seq = rng.standard_normal((N, V))
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    g = rng.standard_normal((N, V))
    bf = oracle.brute_force(seq, cb, T, L, KV, g=g, g_logZ=0.7)
    fd = oracle.finite_difference_grad(seq, cb, T, L, KV, g, 0.7)
    assert np.abs(fd - bf["grad"]).max() < 1e-6 * max(1.0, np.abs(bf["grad"]).max())


@pytest.mark.parametrize("L,KV,V,N,T", [(8, 2, 1, 12, 0.3), (8, 4, 2, 6, 0.8), (10, 2, 1, 16, 0.1)])
def test_reduced_recursion_matches_reference_gather_form(oracle, L, KV, V, N, T):
    """C oracle (reduced state) vs the literal gather+logsumexp restatement."""
    rng = np.random.default_rng(11)
    seq = rng.standard_normal((2, N, V)).astype(np.float32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    soft, logZ = oracle.bcjr_forward(seq, cb, T, L, KV)
    s2, z2, P, la, lb = oracle.naive_forward(seq, cb, T, L, KV, return_internals=True)
    assert np.abs(s2 - soft).max() < 2e-6
    assert np.abs(z2 - logZ).max() < 2e-5 * np.abs(z2).max()
    # invariants: marginals sum to 1, LSE(alpha+beta) = logZ at every step
    assert np.abs(P.sum(-1) - 1.0).max() < 1e-9
    lse = oracle._lse(la + lb, axis=-1)
    assert np.abs(lse - z2[:, None]).max() < 1e-9 * np.abs(z2).max()


def test_high_temperature_limit(oracle):
    """T -> inf: P uniform over all states, soft -> mean codeword (forward_backward.py:39-40)."""
    rng = np.random.default_rng(5)
    L, KV = 8, 2
    cb = rng.standard_normal((1 << L, 1)).astype(np.float32)
    seq = rng.standard_normal((2, 9, 1)).astype(np.float32)
    soft, _ = oracle.bcjr_forward(seq, cb, 1e7, L, KV)
    assert np.abs(soft - cb.mean()).max() < 1e-5


def test_low_temperature_limit_is_viterbi(oracle):
    """T -> 0: soft codeword -> Viterbi reconstruction (forward_backward.py:37-38)."""
    rng = np.random.default_rng(6)
    L, KV = 8, 2
    cb = rng.standard_normal((1 << L, 1)).astype(np.float32)
    seq = rng.standard_normal((3, 20, 1)).astype(np.float32)
    soft, _ = oracle.bcjr_forward(seq, cb, 1e-4, L, KV)
    _, _, _, recon, _ = oracle.viterbi(seq, cb, L, KV)
    assert np.abs(soft - recon).max() < 1e-3


def test_gradient_linear_in_upstream(oracle):
    rng = np.random.default_rng(9)
    L, KV = 8, 2
    cb = rng.standard_normal((1 << L, 1)).astype(np.float32)
    seq = rng.standard_normal((2, 10, 1)).astype(np.float32)
    g1 = rng.standard_normal(seq.shape).astype(np.float32)
    g2 = rng.standard_normal(seq.shape).astype(np.float32)
    d1 = oracle.bcjr_backward(seq, cb, 0.4, L, KV, g1)
    d2 = oracle.bcjr_backward(seq, cb, 0.4, L, KV, g2)
    d12 = oracle.bcjr_backward(seq, cb, 0.4, L, KV, g1 + g2)
    assert max_rel(d1 + d2, d12) < 1e-5


def _entropy(P):
    P = np.asarray(P, dtype=np.float64)
    return -np.where(P > 0, P * np.log(np.where(P > 0, P, 1.0)), 0.0).sum(-1)


@pytest.mark.parametrize("L,KV,V,N,T", TINY[:5])
def test_marginal_entropy_matches_brute_force(oracle, L, KV, V, N, T):
    """-sum P ln P of the path-enumerated marginals (independent of the recursion)."""
    rng = np.random.default_rng(40 + L * 100 + N)
    seq = rng.standard_normal((2, N, V)).astype(np.float32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    H = oracle.marginal_entropy(seq, cb, T, L, KV)
    assert H.shape == (2, N) and H.dtype == np.float32
    for b in range(2):
        bf = oracle.brute_force(seq[b], cb, T, L, KV)
        assert np.abs(H[b] - _entropy(bf["marg"])).max() < 2e-6 * L


def test_marginal_entropy_matches_gather_form(oracle):
    rng = np.random.default_rng(12)
    L, KV, V, N, T = 10, 2, 1, 16, 0.2
    seq = rng.standard_normal((3, N, V)).astype(np.float32)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    _, _, P, _, _ = oracle.naive_forward(seq, cb, T, L, KV, return_internals=True)
    assert np.abs(oracle.marginal_entropy(seq, cb, T, L, KV) - _entropy(P)).max() < 1e-5


def test_marginal_entropy_limits(oracle):
    """T -> inf: every state has the same number of paths, so P_t is uniform and
    H = L ln 2.  T -> 0 with a unique minimum-cost path: H -> 0."""
    rng = np.random.default_rng(13)
    L, KV = 8, 2
    cb = rng.standard_normal((1 << L, 1)).astype(np.float32)
    seq = rng.standard_normal((2, 9, 1)).astype(np.float32)
    assert np.abs(oracle.marginal_entropy(seq, cb, 1e7, L, KV) - L * np.log(2.0)).max() < 1e-5
    assert oracle.marginal_entropy(seq, cb, 1e-4, L, KV).max() < 1e-3


# ------------------------------- Viterbi ---------------------------------

def test_viterbi_toy_known_answer(oracle):
    """src/tripwires/test_viterbi.py:17-53: L=2, k=1 hand-traced walk 00->00->01->11."""
    cb = np.array([-1.2, -0.3, 0.4, 1.1], np.float32)[:, None]
    seq = np.array([-1.0, 0.5, 0.8], np.float32)[None, :, None]
    walk, bits, start, recon, mse = oracle.viterbi(seq, cb, L=2, KV=1)
    assert np.allclose(recon.ravel(), [-1.2, -0.3, 1.1], atol=1e-6)
    assert abs(float(((recon - seq) ** 2).sum()) - 0.77) < 1e-4
    assert walk.tolist() == [[0, 1, 3]] and int(start[0]) == 0 and bits.tolist() == [[0, 1, 1]]


def _f32_path_costs(paths, cb, seq1):
    c = np.zeros(len(paths), np.float32)
    for t in range(seq1.shape[0]):
        d = (cb[paths[:, t]] - seq1[t][None]).astype(np.float32)
        loc = np.zeros(len(paths), np.float32)
        for v in range(seq1.shape[1]):
            loc = (loc + (d[:, v] * d[:, v]).astype(np.float32)).astype(np.float32)
        c = (c + loc).astype(np.float32)
    return c


@pytest.mark.parametrize("L,KV,V,N", [(4, 2, 1, 5), (4, 2, 2, 4), (5, 1, 1, 6), (6, 2, 1, 4), (8, 4, 2, 3)])
def test_viterbi_is_min_cost_path(oracle, L, KV, V, N):
    rng = np.random.default_rng(L + N)
    paths = oracle.enumerate_paths(L, KV, N)
    for _ in range(20):
        cb = rng.standard_normal((1 << L, V)).astype(np.float32)
        seq = rng.standard_normal((1, N, V)).astype(np.float32)
        walk, bits, start, recon, mse = oracle.viterbi(seq, cb, L, KV)
        c = _f32_path_costs(paths, cb, seq[0])
        idx = np.where((paths == walk[0][None]).all(1))[0]
        assert len(idx) == 1 and c[idx[0]] == c.min()
        w2, r2 = oracle.decode(bits, start, cb, L, KV)
        assert (w2 == walk).all() and (r2 == recon).all()


@pytest.mark.parametrize("L,KV,V,N", [(4, 2, 1, 5), (4, 2, 2, 4), (5, 1, 1, 6), (8, 4, 2, 3)])
def test_viterbi_trace_vs_brute_force(oracle, L, KV, V, N):
    """cum_t(s) is the smallest float32 prefix cost over the paths through s at
    step t (fl(x + E) is monotone in x, so the recursion's minimum equals it
    bit for bit) and the backpointer is the lowest predecessor attaining the
    previous step's minimum; the backtrace from the final argmin is the C
    encoder's walk, with its start state."""
    rng = np.random.default_rng(10 * L + N)
    paths = oracle.enumerate_paths(L, KV, N)
    S, R = 1 << L, 1 << KV
    for rep in range(6):
        cb = rng.standard_normal((S, V)).astype(np.float32)
        if rep == 5:
            cb = np.round(cb * 2) / 2  # coarse codewords: ties between predecessors
        seq = rng.standard_normal((1, N, V)).astype(np.float32)
        trace, bp = oracle.viterbi_trace(seq[0], cb, L, KV)
        prefix = np.zeros(len(paths), np.float32)
        best = np.zeros((N, S), np.float32)
        for t in range(N):
            prefix = (prefix + _f32_path_costs(paths[:, t:t + 1], cb, seq[0, t:t + 1])).astype(np.float32)
            b = np.full(S, np.inf, np.float32)
            np.minimum.at(b, paths[:, t], prefix)
            best[t] = b
        assert np.array_equal(trace, best)
        s = np.arange(S)
        assert np.array_equal(bp[0], s >> KV)
        for t in range(1, N):
            preds = (np.arange(R)[None, :] << (L - KV)) | (s[:, None] >> KV)
            costs = best[t - 1][preds]
            want = preds[s, np.argmax(costs == costs.min(axis=1, keepdims=True), axis=1)]
            assert np.array_equal(bp[t], want)
        walk, _, start, _, _ = oracle.viterbi(seq, cb, L, KV)
        w = np.empty(N, np.int64)
        w[-1] = int(np.argmin(trace[-1]))
        for t in range(N - 1, 0, -1):
            w[t - 1] = bp[t, w[t]]
        assert w.tolist() == walk[0].tolist() and int(bp[0, w[0]]) == int(start[0])


def test_viterbi_tie_rules(oracle):
    """All-equal codewords: every path ties.  Lowest p at every step and lowest
    final state give the all-zero walk (encode.py:283-296)."""
    L, KV, N = 4, 2, 5
    cb = np.zeros((1 << L, 1), np.float32)
    seq = np.ones((1, N, 1), np.float32)
    walk, bits, start, _, _ = oracle.viterbi(seq, cb, L, KV)
    assert walk.tolist() == [[0] * N] and int(start[0]) == 0
    # Two tied minima at the last step: the lower state index wins.
    cb = np.full((1 << L, 1), 5.0, np.float32)
    cb[3] = cb[9] = 1.0
    seq = np.ones((1, 1, 1), np.float32)
    walk, _, start, _, _ = oracle.viterbi(seq, cb, L, KV)
    assert int(walk[0, 0]) == 3 and int(start[0]) == 0


def test_viterbi_table1_band_1mad(oracle):
    """Table-1 MSE band for 1MAD at L=16, k=2 (src/tripwires/test_viterbi.py:77-133)."""
    rng = np.random.default_rng(42)
    cb = oracle.codebook(oracle.CODE_1MAD, 16)
    seq = rng.standard_normal((16, 256, 1)).astype(np.float32)
    _, _, _, _, mse = oracle.viterbi(seq, cb, 16, 2)
    assert 0.062 <= float(mse.mean()) <= 0.075


@pytest.mark.parametrize("L,KV,V,N,ob", [(4, 2, 1, 5, 2), (6, 2, 1, 5, 4), (4, 1, 1, 7, 3), (6, 2, 2, 4, 3),
                                         (6, 2, 1, 4, 6), (6, 2, 1, 1, 4)])
def test_constrained_viterbi_matches_brute_force(oracle, L, KV, V, N, ob):
    """The minimum-cost path among those whose first state has top ob bits = v
    and whose last state has bottom ob bits = v (encode.py:328-389), for every v;
    no such path <=> start = -1 (where the reference raises)."""
    rng = np.random.default_rng(L * 31 + N + ob)
    cb = rng.standard_normal((1 << L, V)).astype(np.float32)
    seq1 = rng.standard_normal((N, V)).astype(np.float32)
    paths = oracle.enumerate_paths(L, KV, N)
    cost = ((cb[paths] - seq1[None]) ** 2).sum(axis=(1, 2))
    vals = np.arange(1 << ob)
    walk, _, start, _, _ = oracle.viterbi(np.repeat(seq1[None], len(vals), 0), cb, L, KV,
                                          overlap=vals, overlap_bits=ob)
    m = (1 << ob) - 1
    for i, v in enumerate(vals):
        ok = ((paths[:, 0] >> (L - ob)) == v) & ((paths[:, -1] & m) == v)
        if not ok.any():
            assert start[i] == -1, v
            continue
        best = np.flatnonzero(ok)[np.argmin(cost[ok])]
        assert start[i] == paths[best, 0] >> KV
        assert np.array_equal(walk[i], paths[best]), v


def test_constrained_viterbi_zero_bits_is_unconstrained(oracle):
    rng = np.random.default_rng(14)
    cb = rng.standard_normal((1 << 10, 1)).astype(np.float32)
    seq = rng.standard_normal((3, 40, 1)).astype(np.float32)
    a = oracle.viterbi(seq, cb, 10, 2)
    b = oracle.viterbi(seq, cb, 10, 2, overlap=[0, 0, 0], overlap_bits=0)
    for x, y in zip(a, b):
        assert np.array_equal(x, y)


def test_tailbiting_gate(oracle):
    """The reference's tail-biting gate (test_viterbi.py:135-197) at L=12, k=2,
    1MAD: every walk wraps around (s_0 >> k == s_{N-1} mod 2^(L-k) == overlap)
    and the mean MSE is within 0.005 of the unconstrained encoder's."""
    rng = np.random.default_rng(42)
    L, k = 12, 2
    cb = oracle.codebook(oracle.CODE_1MAD, L)
    seq = rng.standard_normal((32, 256, 1)).astype(np.float32)
    _, _, _, _, mse0 = oracle.viterbi(seq, cb, L, k)
    walk, bits, start, recon, mse, ov = oracle.viterbi_tailbiting(seq, cb, L, k, 1)
    assert (start >= 0).all()
    assert np.array_equal(walk[:, 0] >> k, ov)
    assert np.array_equal(walk[:, -1] & ((1 << (L - k)) - 1), ov)
    assert abs(float(mse.mean()) - float(mse0.mean())) < 0.005


# ------------------------------- codebooks -------------------------------

@pytest.mark.parametrize("name,code", [("1mad", 1), ("3inst", 2), ("hyb", 3)])
def test_codebook_golden(oracle, name, code):
    g = json.load(open(GOLDEN))
    lut = np.random.default_rng(g["hyb_lut_seed"]).standard_normal((512, 2)).astype(np.float32)
    cb = oracle.codebook(code, g["L"], lut=lut if code == 3 else None)
    ref = g["codes"][name]
    assert hashlib.sha256(cb.tobytes()).hexdigest() == ref["sha256_f32"]
    assert cb[np.asarray(g["sample_states"])].view(np.uint32).tolist() == ref["sample_bits"]


@pytest.mark.parametrize("code", [1, 2])
def test_codebook_marginals(oracle, code):
    """src/tripwires/test_codes.py:27-40 bands."""
    cb = oracle.codebook(code, 16)[:, 0]
    assert abs(cb.mean()) < 0.05 and 0.85 < cb.var() < 1.15
    assert 2.6 < stats.kurtosis(cb, fisher=False) < 3.4


def test_pack_roundtrip(oracle):
    rng = np.random.default_rng(0)
    for KV in (1, 2, 4):
        bits = rng.integers(0, 1 << KV, size=(5, 37)).astype(np.int32)
        assert (oracle.unpack_bits(oracle.pack_bits(bits, KV), 37, KV) == bits).all()


def test_pack_layout_known_bytes(oracle):
    # LSB-first: step t occupies bits [t*kV, (t+1)*kV) of the stream
    bits = np.array([[1, 2, 3, 0, 3]], dtype=np.int32)
    assert oracle.pack_bits(bits, 2).tolist() == [[1 | 2 << 2 | 3 << 4 | 0 << 6, 3]]
    bits1 = np.array([[1, 0, 1, 1, 0, 0, 0, 1, 1]], dtype=np.int32)
    assert oracle.pack_bits(bits1, 1).tolist() == [[0b10001101, 0b1]]
    bits4 = np.array([[0xA, 0x3, 0xF]], dtype=np.int32)
    assert oracle.pack_bits(bits4, 4).tolist() == [[0x3A, 0x0F]]


# ---------------------------- Hadamard transform -----------------------------

@pytest.mark.parametrize("n", [1, 2, 8, 64, 512])
def test_fwht_is_sylvester_hadamard_product(oracle, n):
    from scipy.linalg import hadamard
    rng = np.random.default_rng(n)
    Hm = hadamard(n).astype(np.float64)
    xi = rng.integers(-50, 50, size=(3, n)).astype(np.float32)  # integer sums are exact in float32
    assert np.array_equal(oracle.fwht(xi), (xi.astype(np.float64) @ Hm.T).astype(np.float32))
    xf = rng.standard_normal((3, n)).astype(np.float32)
    ref = xf.astype(np.float64) @ Hm.T
    assert np.abs(oracle.fwht(xf) - ref).max() <= 1e-5 * max(1.0, np.abs(ref).max())


@pytest.mark.parametrize("m,n", [(4, 8), (64, 32), (16, 256)])
def test_rht_matches_matrix_form_and_inverts(oracle, m, n):
    from scipy.linalg import hadamard
    rng = np.random.default_rng(m * n)
    W = rng.standard_normal((m, n)).astype(np.float32)
    sl = rng.choice([-1.0, 1.0], size=m).astype(np.float32)
    sr = rng.choice([-1.0, 1.0], size=n).astype(np.float32)
    Hm, Hn = hadamard(m).astype(np.float64), hadamard(n).astype(np.float64)
    ref = Hm @ np.diag(sl) @ W.astype(np.float64) @ np.diag(sr) @ Hn / np.sqrt(m * n)
    Wt = oracle.rht(W, sl, sr)
    assert np.abs(Wt - ref).max() <= 1e-5 * np.abs(ref).max()
    inv_ref = np.diag(sl) @ Hm @ ref @ Hn @ np.diag(sr) / np.sqrt(m * n)
    assert np.abs(inv_ref - W).max() <= 1e-9 * np.abs(W).max() + 1e-12   # the matrix form itself inverts
    back = oracle.inverse_rht(Wt, sl, sr)
    assert np.abs(back - W).max() <= 1e-5 * np.abs(W).max()
    assert abs(np.linalg.norm(Wt) - np.linalg.norm(W)) <= 1e-5 * np.linalg.norm(W)  # orthogonal


def test_torch_eager_restatement_matches_oracle(oracle):
    """oracle/torch_ref.py (the reference's eager node in torch float32, the CPU
    baseline of bench.py) against the float64 C oracle: soft, log Z and the
    gradient, V = 1 and V = 2, with and without the per-step checkpoint."""
    import torch
    from oracle.torch_ref import eager_bcjr, eager_step
    for L, kV, V, code in ((8, 2, 1, oracle.CODE_1MAD), (8, 4, 2, None)):
        rng = np.random.default_rng(L + kV)
        B, N = 3, 24
        seq = rng.standard_normal((B, N, V)).astype(np.float32)
        g = rng.standard_normal((B, N, V)).astype(np.float32)
        cb = oracle.codebook(code, L) if code else rng.standard_normal((1 << L, V)).astype(np.float32)
        s, z, d = eager_step(torch.tensor(seq), torch.tensor(cb), 0.2, L, kV, torch.tensor(g))
        s_ref, z_ref = oracle.bcjr_forward(seq, cb, 0.2, L, kV)
        d_ref = oracle.bcjr_backward(seq, cb, 0.2, L, kV, g)
        assert np.abs(s.numpy() - s_ref).max() <= 1e-4 * np.abs(s_ref).max()
        assert np.abs(z.numpy() - z_ref).max() <= 1e-5 * np.abs(z_ref).max()
        assert np.abs(d.numpy() - d_ref).max() <= 1e-3 * np.abs(d_ref).max()
        x = torch.tensor(seq, requires_grad=True)
        s2, _ = eager_bcjr(x, torch.tensor(cb), 0.2, L, kV, checkpoint=False)
        s2.backward(torch.tensor(g))
        assert torch.allclose(s2.detach(), s, rtol=0, atol=1e-6) and torch.allclose(x.grad, d, rtol=0, atol=1e-5)


@pytest.mark.parametrize("kV,V,N,code,T", [(2, 1, 256, "3inst", 0.1), (4, 2, 128, "hyb", 0.3)])
def test_oracle_at_l16_matches_float64_gather_form(oracle, kV, V, N, code, T):
    """The C oracle at the headline trellis size, L = 16 (65,536 states), one
    tile, against oracle/torch_ref.py's literal gather form run in float64 (the
    reference's eager node, src/bcjr/forward_backward.py:89-232, every state
    gathering its 2^kV predecessors; autograd for the gradient).  kV = 2 with
    the 3INST code at N = 256 (the layer's trellis) and kV = 4 with a HYB Q = 9
    table at N = 128 (the reference's QAT trellis).  The two share no code, so
    an L-dependent mistake in the structure-aware oracle -- a shift or mask
    width, a reduced-state index, 32-bit index arithmetic over 2^16 x 256 cells
    -- fails here; the tolerances are the float32 rounding of the oracle's
    outputs, 100-1000 times tighter than the parity gates."""
    import torch
    from oracle.torch_ref import eager_step
    L = 16
    rng = np.random.default_rng(16 + kV)
    seq = rng.standard_normal((1, N, V)).astype(np.float32)
    g = rng.standard_normal((1, N, V)).astype(np.float32)
    if code == "hyb":
        cb = oracle.codebook(oracle.CODE_HYB, L, lut=rng.standard_normal((512, 2)).astype(np.float32), Q=9)
    else:
        cb = oracle.codebook(oracle.CODE_3INST, L)
    f64 = lambda a: torch.tensor(a, dtype=torch.float64)  # noqa: E731
    s, z, d = eager_step(f64(seq), f64(cb), T, L, kV, f64(g))
    s_ref, z_ref = oracle.bcjr_forward(seq, cb, T, L, kV)
    d_ref = oracle.bcjr_backward(seq, cb, T, L, kV, g)
    assert np.abs(s.numpy() - s_ref).max() <= 1e-6 * np.abs(s_ref).max()
    assert np.abs(z.numpy() - z_ref).max() <= 1e-6 * np.abs(z_ref).max()
    assert np.abs(d.numpy() - d_ref).max() <= 1e-5 * np.abs(d_ref).max()
