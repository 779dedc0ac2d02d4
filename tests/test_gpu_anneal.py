"""GPU parity of the fused marginal entropy (bcjr_forward_entropy through the C
ABI) and the annealing helpers of src/bcjr/anneal.py.

H[b, t] = -sum_s P_t(s) ln P_t(s) in nats against the oracle's float64 value
(itself pinned by path enumeration and the gather form), against P from
return_internals, and at the T -> inf closed form L ln 2; entropy_diagnostic
over a layer against the oracle mean of the same tiles.
Bar: |H - H_ref| <= 1e-4 * max(1, max H_ref); soft and log Z of the same launch
as for bcjr_forward."""
import math

import numpy as np
import pytest
import torch

from conftest import max_rel

pytestmark = pytest.mark.gpu

H_TOL = 1e-4


def _say(msg):
    print(msg, flush=True)


def _codebook(bcjr, kind, L, rng):
    if kind == "table":
        cb = torch.tensor(rng.standard_normal((1 << L, 1)).astype(np.float32), device="cuda")
    elif kind == "table2":
        cb = torch.tensor(rng.standard_normal((1 << L, 2)).astype(np.float32), device="cuda")
    elif kind == "1mad":
        cb = bcjr.make_1mad_codebook(L, "cuda")
    elif kind == "3inst":
        cb = bcjr.make_3inst_codebook(L, "cuda")
    elif kind == "hyb":
        lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
        cb = bcjr.make_hyb_codebook_gpu(lut, Q=9, L_bits=L, device="cuda")
    else:
        raise ValueError(kind)
    return cb, cb.cpu().numpy()


def _h_close(H, H_ref):
    H = np.asarray(H, dtype=np.float64)
    return np.abs(H - H_ref).max() <= H_TOL * max(1.0, float(np.abs(H_ref).max()))


# (L, k, V, N, B, codebook, T)
CASES = [
    (8, 2, 1, 12, 3, "table", 0.3),
    (10, 1, 1, 64, 4, "table", 0.2),       # kV = 1
    (12, 2, 1, 256, 4, "1mad", 0.1),
    (12, 2, 2, 128, 3, "hyb", 0.3),        # kV = 4
    (12, 2, 2, 64, 2, "table2", 0.5),
    (16, 2, 1, 256, 2, "3inst", 0.1),      # single-tile config
    (16, 2, 1, 128, 2, "3inst", 0.05),     # below 0.08: group-maximum variant
    (16, 2, 2, 64, 2, "hyb", 0.1),         # reference QAT trellis (kV = 4)
]


@pytest.mark.parametrize("L,k,V,N,B,kind,T", CASES)
def test_marginal_entropy_vs_oracle(bcjr_mod, oracle, L, k, V, N, B, kind, T):
    _say(f"entropy L={L} k={k} V={V} N={N} B={B} {kind} T={T}")
    from bcjr import ops
    from bcjr.codes import resolve_codebook
    rng = np.random.default_rng(L * 7 + N)
    cb, cb_np = _codebook(bcjr_mod, kind, L, rng)
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    H = bcjr_mod.bcjr_marginal_entropy(torch.tensor(seq, device="cuda"), cb, T, L=L, k=k, V=V)
    assert H.shape == (B, N) and H.dtype == torch.float32
    H_ref = oracle.marginal_entropy(seq, cb_np, T, L, k * V)
    assert _h_close(H.cpu().numpy(), H_ref)
    # soft and log Z of the entropy launch are those of the plain forward
    spec, table = resolve_codebook(cb, L, k, V, torch.device("cuda"))
    s1, z1, _ = ops.forward_entropy(spec, torch.tensor(seq, device="cuda"), T, table)
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, T, L, k * V)
    assert max_rel(s1.cpu().numpy(), s_ref) < 1e-4
    assert np.abs(z1.cpu().numpy() - z_ref).max() <= 1e-5 * np.abs(z_ref).max()


def test_marginal_entropy_per_sequence_temperature(bcjr_mod, oracle):
    _say("entropy per-sequence T")
    rng = np.random.default_rng(3)
    L, N = 12, 64
    cb, cb_np = _codebook(bcjr_mod, "1mad", L, rng)
    seq = rng.standard_normal((4, N, 1)).astype(np.float32)
    Ts = np.array([0.05, 0.2, 1.0, 5.0], dtype=np.float32)
    H = bcjr_mod.bcjr_marginal_entropy(torch.tensor(seq, device="cuda"), cb, torch.tensor(Ts, device="cuda"),
                                       L=L, k=2, V=1)
    assert _h_close(H.cpu().numpy(), oracle.marginal_entropy(seq, cb_np, Ts, L, 2))
    # higher temperature, flatter marginals
    assert (H.mean(dim=1).diff() > 0).all()


def test_marginal_entropy_matches_internals(bcjr_mod):
    """H from the fused output equals -sum P ln P of the marginals that
    return_internals materialises (the reference's entropy_diagnostic body)."""
    _say("entropy vs return_internals")
    rng = np.random.default_rng(8)
    L, N = 10, 32
    cb, _ = _codebook(bcjr_mod, "table", L, rng)
    seq = torch.tensor(rng.standard_normal((3, N, 1)).astype(np.float32), device="cuda")
    _, _, P, _, _ = bcjr_mod.bcjr_forward_backward(seq, cb, 0.3, L=L, k=2, V=1, return_internals=True)
    logP = P.clamp(min=1e-30).log()
    H_ref = -(P * logP).sum(dim=-1)
    H = bcjr_mod.bcjr_marginal_entropy(seq, cb, 0.3, L=L, k=2, V=1)
    assert _h_close(H.cpu().numpy(), H_ref.double().cpu().numpy())


def test_marginal_entropy_high_temperature_is_uniform(bcjr_mod):
    """T -> inf: every state lies on equally many paths, so H = L ln 2 at every
    step, at the full single-tile size (L=16, N=256, 64 sequences)."""
    _say("entropy T -> inf, L=16")
    rng = np.random.default_rng(4)
    cb, _ = _codebook(bcjr_mod, "3inst", 16, rng)
    seq = torch.tensor(rng.standard_normal((64, 256, 1)).astype(np.float32), device="cuda")
    H = bcjr_mod.bcjr_marginal_entropy(seq, cb, 1e6, L=16, k=2, V=1)
    assert (H - 16 * math.log(2.0)).abs().max() < 1e-3
    Hc = bcjr_mod.bcjr_marginal_entropy(seq, cb, 0.1, L=16, k=2, V=1)
    assert (Hc >= -1e-4).all() and (Hc <= 16 * math.log(2.0) + 1e-3).all()


def test_entropy_diagnostic_over_a_layer(bcjr_mod, oracle):
    """entropy_diagnostic on two quantized linears (one in STE mode, skipped):
    the mean over every tile (max_tiles=None) against the oracle mean of the same
    rotated, normalised tiles; a sampled draw stays within the per-tile range."""
    from types import SimpleNamespace
    from bcjr.quant import tile_for_viterbi
    _say("entropy_diagnostic")
    rng = np.random.default_rng(5)
    L = 12
    cb, cb_np = _codebook(bcjr_mod, "1mad", L, rng)
    T = torch.tensor(0.2, device="cuda")

    def ql(m, n, seed, mode="bcjr"):
        r = np.random.default_rng(seed)
        return SimpleNamespace(W_latent=torch.tensor(r.standard_normal((m, n)).astype(np.float32) * 0.02,
                                                     device="cuda"),
                               sign_l=torch.tensor(r.choice([-1.0, 1.0], m).astype(np.float32), device="cuda"),
                               sign_r=torch.tensor(r.choice([-1.0, 1.0], n).astype(np.float32), device="cuda"),
                               codebook_gpu=cb, T_temp=T, quant_mode=mode)

    qls = [ql(64, 64, 1), ql(32, 128, 2), ql(64, 32, 3, mode="ste")]
    got = bcjr_mod.entropy_diagnostic(qls, max_tiles=None)
    tot, cnt = 0.0, 0
    for q in qls[:2]:
        Wt = bcjr_mod.apply_rht_gpu(q.W_latent, q.sign_l, q.sign_r)
        unit = Wt / Wt.pow(2).mean().sqrt()
        seqs, _ = tile_for_viterbi(unit, 16, 16)
        seqs = seqs.cpu().numpy().reshape(seqs.shape[0], 256, 1)
        H = oracle.marginal_entropy(seqs, cb_np, 0.2, L, 2)
        tot += float(H.astype(np.float64).sum())
        cnt += H.size
    assert abs(got - tot / cnt) <= H_TOL * max(1.0, tot / cnt)
    g = torch.Generator(device="cuda")
    g.manual_seed(0)
    sampled = bcjr_mod.entropy_diagnostic(qls, max_tiles=4, generator=g)
    assert 0.0 <= sampled <= L * math.log(2.0)
    assert math.isnan(bcjr_mod.entropy_diagnostic(qls[2:]))

