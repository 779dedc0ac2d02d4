"""GPU parity of the expert-batched dispatch: the batched RHT against the oracle
transform of each matrix, and bcjr_quantize_experts (one engine call for many
weights, per-weight temperatures) against the oracle composition of RHT, BCJR
and inverse RHT on each weight, and against per-weight bcjr_quantize_weight
calls (the reference's per-expert loop, src/qat/qat_moe_layer.py:106-114)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu

SOFT_TOL = 1e-4
GRAD_TOL = 1e-3


def _say(msg):
    print(msg, flush=True)


def _signs(n, seed):
    return np.random.default_rng(seed).choice([-1.0, 1.0], size=n).astype(np.float32)


# m*n an even power of two: the scale 1/sqrt(mn) is exact, so the match is bit-exact
@pytest.mark.parametrize("E,m,n", [(3, 64, 256), (5, 256, 16), (2, 2048, 512), (4, 1, 64)])
def test_rht_batched_bit_exact(bcjr_mod, oracle, E, m, n):
    _say(f"rht batched E={E} {m}x{n}")
    rng = np.random.default_rng(E * m + n)
    W = rng.standard_normal((E, m, n)).astype(np.float32)
    SL = np.stack([_signs(m, 10 + e) for e in range(E)])
    SR = np.stack([_signs(n, 50 + e) for e in range(E)])
    Wd, sl, sr = (torch.tensor(a, device="cuda") for a in (W, SL, SR))
    Wt = bcjr_mod.apply_rht_batched(Wd, sl, sr)
    back = bcjr_mod.apply_inverse_rht_batched(Wt, sl, sr)
    for e in range(E):
        assert np.array_equal(Wt[e].cpu().numpy(), oracle.rht(W[e], SL[e], SR[e]))
        assert np.array_equal(back[e].cpu().numpy(), oracle.inverse_rht(Wt[e].cpu().numpy(), SL[e], SR[e]))
        # the single-matrix entry point gives the same bits
        assert torch.equal(Wt[e], bcjr_mod.apply_rht_gpu(Wd[e], sl[e], sr[e]))


def test_rht_batched_gradient_is_adjoint(bcjr_mod):
    _say("rht batched adjoint")
    E, m, n = 3, 64, 32
    W = torch.randn(E, m, n, device="cuda", requires_grad=True)
    g = torch.randn(E, m, n, device="cuda")
    sl = torch.tensor(np.stack([_signs(m, e) for e in range(E)]), device="cuda")
    sr = torch.tensor(np.stack([_signs(n, 9 + e) for e in range(E)]), device="cuda")
    (bcjr_mod.apply_rht_batched(W, sl, sr) * g).sum().backward()
    assert torch.equal(W.grad, bcjr_mod.apply_inverse_rht_batched(g, sl, sr))


def _weights(shapes, seed):
    rng = np.random.default_rng(seed)
    Ws = [(rng.standard_normal(s) * 0.02).astype(np.float32) for s in shapes]
    SL = [_signs(s[0], seed + 2 * i) for i, s in enumerate(shapes)]
    SR = [_signs(s[1], seed + 2 * i + 1) for i, s in enumerate(shapes)]
    return Ws, SL, SR


def test_experts_match_oracle_composition(bcjr_mod, oracle):
    """Four weights of two shapes with four temperatures in one call; every weight
    against RHT -> RMS scale -> tiles -> BCJR at its T -> untile -> inverse RHT on
    the oracle, values and gradients."""
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    _say("experts vs oracle, L=12 1MAD")
    L, k, V = 12, 2, 1
    shapes = [(64, 128), (128, 64), (64, 128), (128, 64)]
    Ts = [0.1, 0.05, 0.3, 0.1]
    Ws, SL, SR = _weights(shapes, 7)
    cb = bcjr_mod.make_1mad_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    Wd = [torch.tensor(W, device="cuda", requires_grad=True) for W in Ws]
    outs = bcjr_mod.bcjr_quantize_experts(Wd, [torch.tensor(s, device="cuda") for s in SL],
                                          [torch.tensor(s, device="cuda") for s in SR], cb, Ts, L=L, k=k, V=V)
    rng = np.random.default_rng(99)
    gs = [rng.standard_normal(s).astype(np.float32) for s in shapes]
    sum((o * torch.tensor(g, device="cuda")).sum() for o, g in zip(outs, gs)).backward()
    for e, (W, sl, sr, T, g) in enumerate(zip(Ws, SL, SR, Ts, gs)):
        m, n = W.shape
        Wt = oracle.rht(W, sl, sr)
        scale = np.float32(np.sqrt((Wt ** 2).mean(dtype=np.float32)))
        seqs, info = tile_for_viterbi(torch.tensor(Wt / scale), 16, 16)
        seqs = seqs.numpy().reshape(seqs.shape[0], -1, V)
        soft, _ = oracle.bcjr_forward(seqs, cb_np, T, L, k * V)
        Wtq = untile_from_viterbi(torch.tensor(soft.reshape(seqs.shape[0], -1)), info, (m, n), 16, 16).numpy()
        ref = oracle.inverse_rht(Wtq * scale, sl, sr)
        got = outs[e].detach().cpu().numpy()
        assert np.abs(got - ref).max() <= SOFT_TOL * np.abs(ref).max(), e
        gt = oracle.rht(g, sl, sr)
        gt_tiles, _ = tile_for_viterbi(torch.tensor(gt * scale), 16, 16)
        d_seq = oracle.bcjr_backward(seqs, cb_np, T, L, k * V, gt_tiles.numpy().reshape(seqs.shape))
        d_wt = untile_from_viterbi(torch.tensor(d_seq.reshape(seqs.shape[0], -1) / scale), info, (m, n),
                                   16, 16).numpy()
        grad_ref = oracle.inverse_rht(d_wt, sl, sr)
        assert np.abs(Wd[e].grad.cpu().numpy() - grad_ref).max() <= GRAD_TOL * np.abs(grad_ref).max(), e


def test_experts_match_per_weight_loop(bcjr_mod):
    """The batched call against one bcjr_quantize_weight per weight (the reference's
    loop) on OLMoE-proportioned shapes (gate_up 2I x H, down H x I at 1/16 scale),
    HYB L=16; the per-weight scale is a float32 reduction in both, so the match is
    to the soft tolerance."""
    _say("experts vs per-weight loop, HYB L=16")
    lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr_mod.make_hyb_codebook_gpu(lut, 9, 16, "cuda")
    H, I = 128, 64
    shapes = [(2 * I, H), (H, I)] * 3
    Ts = torch.tensor([0.2, 0.2, 0.1, 0.1, 0.05, 0.05], device="cuda")
    Ws, SL, SR = _weights(shapes, 31)
    Wd = [torch.tensor(W, device="cuda", requires_grad=True) for W in Ws]
    sl = [torch.tensor(s, device="cuda") for s in SL]
    sr = [torch.tensor(s, device="cuda") for s in SR]
    outs = bcjr_mod.bcjr_quantize_experts(Wd, sl, sr, cb, Ts)
    gs = [torch.randn(s, device="cuda") for s in shapes]
    sum((o * g).sum() for o, g in zip(outs, gs)).backward()
    for e in range(len(shapes)):
        W1 = torch.tensor(Ws[e], device="cuda", requires_grad=True)
        ref = bcjr_mod.bcjr_quantize_weight(W1, sl[e], sr[e], cb, Ts[e])
        (ref * gs[e]).sum().backward()
        assert (outs[e] - ref).abs().max() <= SOFT_TOL * ref.abs().max(), e
        assert (Wd[e].grad - W1.grad).abs().max() <= GRAD_TOL * W1.grad.abs().max(), e


def test_moe_dict_form(bcjr_mod):
    _say("experts dict form")
    cb = bcjr_mod.make_3inst_codebook(16, "cuda")
    names = [(e, p) for e in range(2) for p in ("gate_up", "down")]
    shapes = {"gate_up": (64, 32), "down": (32, 32)}
    W = {nm: torch.randn(shapes[nm[1]], device="cuda") * 0.02 for nm in names}
    signs = {nm: (torch.tensor(_signs(shapes[nm[1]][0], i), device="cuda"),
                  torch.tensor(_signs(shapes[nm[1]][1], 40 + i), device="cuda")) for i, nm in enumerate(names)}
    out = bcjr_mod.quantize_moe_experts(W, signs, cb, {nm: 0.1 for nm in names}, L=16, k=2, V=1)
    assert list(out) == names
    for nm in names:
        ref = bcjr_mod.bcjr_quantize_weight(W[nm], signs[nm][0], signs[nm][1], cb, 0.1, L=16, k=2, V=1)
        assert (out[nm] - ref).abs().max() <= SOFT_TOL * ref.abs().max()


def test_ste_experts_bit_exact_vs_oracle(bcjr_mod, oracle):
    """Hard quantization of several weights in one Viterbi launch: every weight
    against RHT -> its RMS scale -> tiles -> Viterbi -> untile -> inverse RHT on
    the oracle, bit for bit (the scale is the same float32 reduction, read back)."""
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    _say("STE experts vs oracle, HYB L=16")
    lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr_mod.make_hyb_codebook_gpu(lut, 9, 16, "cuda")
    shapes = [(64, 256), (256, 64), (64, 256)]
    Ws, SL, SR = _weights(shapes, 41)
    Wd = [torch.tensor(W, device="cuda") for W in Ws]
    sl = [torch.tensor(s, device="cuda") for s in SL]
    sr = [torch.tensor(s, device="cuda") for s in SR]
    outs = bcjr_mod.ste_quantize_experts(Wd, sl, sr, cb)
    cb_np = cb.cpu().numpy()
    for e, (W, a, b) in enumerate(zip(Ws, SL, SR)):
        m, n = W.shape
        Wt = bcjr_mod.apply_rht_batched(Wd[e][None], sl[e][None], sr[e][None])
        s = float(Wt.pow(2).mean(dim=(1, 2)).sqrt()[0])
        Wt_np = oracle.rht(W, a, b)
        assert np.array_equal(Wt[0].cpu().numpy(), Wt_np)
        seqs, info = tile_for_viterbi(torch.tensor(Wt_np / np.float32(s)), 16, 16)
        _, _, _, recon, _ = oracle.viterbi(seqs.numpy().reshape(seqs.shape[0], -1, 2), cb_np, 16, 4)
        q = untile_from_viterbi(torch.tensor(recon.reshape(seqs.shape[0], -1)), info, (m, n), 16, 16).numpy()
        ref = oracle.inverse_rht((q * np.float32(s)).astype(np.float32), a, b)
        assert np.array_equal(outs[e].cpu().numpy(), ref), e


def test_measure_ptq_residual_over_a_layer(bcjr_mod):
    from types import SimpleNamespace
    _say("measure_ptq_residual")
    cb = bcjr_mod.make_3inst_codebook(16, "cuda")
    qls = [SimpleNamespace(W_latent=torch.randn(m, n, device="cuda") * 0.02,
                           sign_l=torch.tensor(_signs(m, i), device="cuda"),
                           sign_r=torch.tensor(_signs(n, 10 + i), device="cuda"), codebook_gpu=cb)
           for i, (m, n) in enumerate([(64, 64), (128, 64)])]
    tot, cnt = 0.0, 0
    for ql in qls:
        ssq, c = bcjr_mod.ptq_residual(ql.W_latent, ql.sign_l, ql.sign_r, cb)
        tot, cnt = tot + ssq, cnt + c
    assert bcjr_mod.measure_ptq_residual(qls) == tot / cnt
    assert bcjr_mod.measure_ptq_residual(qls[0]) == bcjr_mod.ptq_residual(qls[0].W_latent, qls[0].sign_l,
                                                                         qls[0].sign_r, cb)[0] / (64 * 64)
