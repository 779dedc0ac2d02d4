"""GPU parity of the Hadamard / RHT kernels against the oracle (src/rht/transform.py
restated), and the RHT-wrapped quantizer (src/bcjr/bcjr_quant.py:159-178) against
the oracle composition of transform, BCJR and inverse transform."""
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


@pytest.mark.parametrize("rows,n", [(5, 1), (3, 2), (7, 64), (33, 256), (16, 2048), (4, 8192), (2, 16384)])
def test_hadamard_bit_exact(bcjr_mod, oracle, rows, n):
    _say(f"hadamard rows={rows} n={n}")
    x = np.random.default_rng(n).standard_normal((rows, n)).astype(np.float32)
    y = bcjr_mod.hadamard_transform(torch.tensor(x, device="cuda"))
    assert np.array_equal(y.cpu().numpy(), oracle.fwht(x))
    y2 = bcjr_mod.hadamard_transform(torch.tensor(x, device="cuda"), scale=0.25)
    assert np.array_equal(y2.cpu().numpy(), oracle.fwht(x) * np.float32(0.25))


def test_hadamard_batched_shape_and_grad(bcjr_mod, oracle):
    _say("hadamard 3-D + grad")
    x = torch.randn(2, 3, 128, device="cuda", requires_grad=True)
    g = torch.randn(2, 3, 128, device="cuda")
    y = bcjr_mod.hadamard_transform(x, scale=0.5)
    (y * g).sum().backward()
    assert y.shape == x.shape
    assert np.array_equal(y.detach().cpu().numpy().reshape(6, 128),
                          oracle.fwht(x.detach().cpu().numpy().reshape(6, 128)) * np.float32(0.5))
    # H is symmetric: the gradient is the same transform of g
    assert np.array_equal(x.grad.cpu().numpy().reshape(6, 128),
                          oracle.fwht(g.cpu().numpy().reshape(6, 128)) * np.float32(0.5))


# (m, n) with m*n an even power of two: the scale is exact and results are bit-exact
EXACT = [(1, 64), (64, 64), (4, 16), (256, 256), (512, 2048), (2048, 512), (128, 8192), (16384, 64), (64, 1)]


@pytest.mark.parametrize("m,n", EXACT)
def test_rht_bit_exact(bcjr_mod, oracle, m, n):
    _say(f"rht m={m} n={n}")
    rng = np.random.default_rng(m + n)
    W = rng.standard_normal((m, n)).astype(np.float32)
    sl, sr = _signs(m, 1), _signs(n, 2)
    Wt = bcjr_mod.apply_rht_gpu(torch.tensor(W, device="cuda"), torch.tensor(sl, device="cuda"),
                                torch.tensor(sr, device="cuda"))
    ref = oracle.rht(W, sl, sr)
    assert np.array_equal(Wt.cpu().numpy(), ref)
    back = bcjr_mod.apply_inverse_rht_gpu(Wt, torch.tensor(sl, device="cuda"), torch.tensor(sr, device="cuda"))
    assert np.array_equal(back.cpu().numpy(), oracle.inverse_rht(ref, sl, sr))
    assert np.abs(back.cpu().numpy() - W).max() <= 1e-5 * np.abs(W).max()


@pytest.mark.parametrize("m,n", [(2, 64), (128, 256), (2048, 64)])
def test_rht_odd_power_scale(bcjr_mod, oracle, m, n):
    """m*n an odd power of two: 1/sqrt(mn) is inexact; float32 multiply vs the
    reference's float64 division differ by at most one rounding."""
    _say(f"rht odd m={m} n={n}")
    W = np.random.default_rng(3).standard_normal((m, n)).astype(np.float32)
    sl, sr = _signs(m, 4), _signs(n, 5)
    Wt = bcjr_mod.apply_rht_gpu(torch.tensor(W, device="cuda"), torch.tensor(sl, device="cuda"),
                                torch.tensor(sr, device="cuda")).cpu().numpy()
    ref = oracle.rht(W, sl, sr)
    assert np.abs(Wt - ref).max() <= 2 * np.spacing(np.abs(ref).max())


def test_rht_adjoint_is_inverse(bcjr_mod):
    """<RHT(W), G> = <W, RHT^-1(G)>, and autograd's gradient of RHT is RHT^-1."""
    _say("rht adjoint")
    m, n = 256, 512
    W = torch.randn(m, n, device="cuda", dtype=torch.float32, requires_grad=True)
    G = torch.randn(m, n, device="cuda")
    sl = torch.tensor(_signs(m, 6), device="cuda")
    sr = torch.tensor(_signs(n, 7), device="cuda")
    Wt = bcjr_mod.apply_rht_gpu(W, sl, sr)
    lhs = float((Wt.detach().double() * G.double()).sum())
    rhs = float((W.detach().double() * bcjr_mod.apply_inverse_rht_gpu(G, sl, sr).double()).sum())
    assert abs(lhs - rhs) <= 1e-4 * max(1.0, abs(lhs))
    (Wt * G).sum().backward()
    assert torch.equal(W.grad, bcjr_mod.apply_inverse_rht_gpu(G, sl, sr))


def test_quantize_weight_vs_oracle_composition(bcjr_mod, oracle):
    """bcjr_quantize_weight (RHT -> RMS scale -> 16x16 tiles -> BCJR soft -> back) and its
    gradient against the same steps on the oracle."""
    _say("quantize_weight with RHT, L=12 1MAD T=0.1")
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    L, k, V, T = 12, 2, 1, 0.1
    m, n = 64, 256
    rng = np.random.default_rng(11)
    W = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
    g = rng.standard_normal((m, n)).astype(np.float32)
    sl, sr = _signs(m, 8), _signs(n, 9)
    cb = bcjr_mod.make_1mad_codebook(L, "cuda")
    cb_np = cb.cpu().numpy()
    Wd = torch.tensor(W, device="cuda", requires_grad=True)
    Wq = bcjr_mod.bcjr_quantize_weight(Wd, torch.tensor(sl, device="cuda"), torch.tensor(sr, device="cuda"),
                                       cb, T, L=L, k=k, V=V)
    (Wq * torch.tensor(g, device="cuda")).sum().backward()

    # oracle composition
    Wt = oracle.rht(W, sl, sr)
    scale = np.float32(np.sqrt((Wt.astype(np.float32) ** 2).mean(dtype=np.float32)))
    seqs, info = tile_for_viterbi(torch.tensor(Wt / scale), 16, 16)
    seqs = seqs.numpy().reshape(seqs.shape[0], -1, V)
    soft, _ = oracle.bcjr_forward(seqs, cb_np, T, L, k * V)
    Wtq = untile_from_viterbi(torch.tensor(soft.reshape(seqs.shape[0], -1)), info, (m, n), 16, 16).numpy()
    ref = oracle.inverse_rht(Wtq * scale, sl, sr)
    got = Wq.detach().cpu().numpy()
    assert np.abs(got - ref).max() <= SOFT_TOL * np.abs(ref).max()

    # gradient: W_q = R^-1(s * U(soft(T(R(W)) / s))) with s detached
    gt = oracle.rht(g, sl, sr)  # adjoint of R^-1 is R
    gt_tiles, _ = tile_for_viterbi(torch.tensor(gt * scale), 16, 16)
    d_seq = oracle.bcjr_backward(seqs, cb_np, T, L, k * V, gt_tiles.numpy().reshape(seqs.shape))
    d_wt = untile_from_viterbi(torch.tensor(d_seq.reshape(seqs.shape[0], -1) / scale), info, (m, n), 16, 16).numpy()
    grad_ref = oracle.inverse_rht(d_wt, sl, sr)  # adjoint of R is R^-1
    assert np.abs(Wd.grad.cpu().numpy() - grad_ref).max() <= GRAD_TOL * np.abs(grad_ref).max()


# ------------------------------ hard STE path --------------------------------

def _hyb_codebook(bcjr_mod, L=16, Q=9):
    lut = np.random.default_rng(2).standard_normal((1 << Q, 2)).astype(np.float32)
    return bcjr_mod.make_hyb_codebook_gpu(lut, Q, L, "cuda")


@pytest.mark.parametrize("codebook_kind,m,n", [("hyb16", 64, 256), ("3inst16", 128, 128), ("1mad12", 512, 32)])
def test_ste_forward_matches_oracle_viterbi(bcjr_mod, oracle, codebook_kind, m, n):
    """TrellisQuantSTE: W_q = R^-1(s * untile(Viterbi recon(tile(R(W) / s)))), bit-exact in
    every step against the oracle (the scale s is read back from the device, since
    it is a float32 reduction)."""
    _say(f"STE {codebook_kind} {m}x{n}")
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    cb = {"hyb16": lambda: _hyb_codebook(bcjr_mod), "3inst16": lambda: bcjr_mod.make_3inst_codebook(16, "cuda"),
          "1mad12": lambda: bcjr_mod.make_1mad_codebook(12, "cuda")}[codebook_kind]()
    L = int(cb.shape[0]).bit_length() - 1
    V = cb.shape[1]
    rng = np.random.default_rng(m * n)
    W = (rng.standard_normal((m, n)) * 0.05).astype(np.float32)
    sl, sr = _signs(m, 12), _signs(n, 13)
    Wd = torch.tensor(W, device="cuda", requires_grad=True)
    Wq = bcjr_mod.TrellisQuantSTE.apply(Wd, torch.tensor(sl, device="cuda"), torch.tensor(sr, device="cuda"), cb)
    g = torch.randn(m, n, device="cuda")
    (Wq * g).sum().backward()
    assert torch.equal(Wd.grad, g)  # straight through

    Wt_gpu = bcjr_mod.apply_rht_gpu(torch.tensor(W, device="cuda"), torch.tensor(sl, device="cuda"),
                                    torch.tensor(sr, device="cuda"))
    s = Wt_gpu.pow(2).mean().sqrt().clamp(min=1e-30)
    unit = (Wt_gpu / s).cpu()
    seqs, info = tile_for_viterbi(unit, 16, 16)
    _, _, _, recon, _ = oracle.viterbi(seqs.numpy().reshape(seqs.shape[0], -1, V), cb.cpu().numpy(), L, 2 * V)
    Wtq = untile_from_viterbi(torch.tensor(recon.reshape(seqs.shape[0], -1)), info, (m, n), 16, 16)
    ref = oracle.inverse_rht((Wtq * s.cpu()).numpy(), sl, sr)
    assert np.array_equal(Wq.detach().cpu().numpy(), ref)


def test_ste_ip_and_walk_replay(bcjr_mod, oracle):
    _say("STE IP + replay walks")
    cb = bcjr_mod.make_3inst_codebook(16, "cuda")
    W = torch.randn(64, 64, device="cuda") * 0.1
    Wq = bcjr_mod.TrellisQuantSTE_IP.apply(W, cb)
    s = W.pow(2).mean().sqrt()
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    seqs, info = tile_for_viterbi(W / s, 16, 16)
    bits, start, recon, _ = bcjr_mod.viterbi_encode_v_batched_hip(seqs.contiguous(), cb, L=16, k=2, V=1)
    assert torch.equal(Wq, untile_from_viterbi(recon, info, (64, 64), 16, 16) * s)
    walks = bcjr_mod.replay_walks(bits.cpu().numpy(), start.cpu().numpy(), L=16, kV=2)
    walk_dec, _ = bcjr_mod.viterbi_decode_v_batched(bits, start, cb, L=16, k=2, V=1)
    assert np.array_equal(walks, walk_dec.cpu().numpy().astype(np.int64))


def test_ptq_residual_definition(bcjr_mod):
    _say("ptq residual")
    cb = bcjr_mod.make_3inst_codebook(16, "cuda")
    m, n = 128, 128
    W = torch.randn(m, n, device="cuda") * 0.02
    sl = torch.tensor(_signs(m, 14), device="cuda")
    sr = torch.tensor(_signs(n, 15), device="cuda")
    ssq, cnt = bcjr_mod.ptq_residual(W, sl, sr, cb)
    assert cnt == m * n
    Wt = bcjr_mod.apply_rht_gpu(W, sl, sr)
    s = Wt.pow(2).mean().sqrt()
    Wq = bcjr_mod.quantize_forward_gpu(W, sl, sr, cb)
    ref = float(((Wt / s - bcjr_mod.apply_rht_gpu(Wq, sl, sr) / s) ** 2).sum())
    assert abs(ssq - ref) <= 1e-5 * ref
    # 2-bit 3INST on unit-variance Gaussians: MSE in the published band (QTIP Table 1 ~0.069)
    assert 0.04 < ssq / cnt < 0.12


def test_rht_and_dequant_capture_replays(bcjr_mod, oracle):
    """The RHT (single and batched) and the dequant kernel captured in one HIP
    graph replay to the eager results, with eager work between replays (the
    entry points are stream-ordered and allocate nothing)."""
    _say("rht + dequant graph capture")
    from bcjr import ops
    from bcjr.serialize import pack_bitstreams
    m, n = 256, 512
    rng = np.random.default_rng(21)
    W = torch.tensor(rng.standard_normal((m, n)).astype(np.float32), device="cuda")
    Wb = torch.tensor(rng.standard_normal((3, 64, 128)).astype(np.float32), device="cuda")
    sl, sr = torch.tensor(_signs(m, 1), device="cuda"), torch.tensor(_signs(n, 2), device="cuda")
    slb = torch.tensor(np.stack([_signs(64, 3 + e) for e in range(3)]), device="cuda")
    srb = torch.tensor(np.stack([_signs(128, 9 + e) for e in range(3)]), device="cuda")
    B = (m // 16) * (n // 16)
    bits = rng.integers(0, 16, (B, 128)).astype(np.uint8)
    packed = torch.tensor(pack_bitstreams(bits, 4), device="cuda")
    start = torch.tensor(rng.integers(0, 1 << 16, B).astype(np.int32), device="cuda")
    lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr_mod.make_hyb_codebook_gpu(lut, 9, 16, "cuda")
    spec = ops.Spec(16, 2, 2, ops.CODE_HYB, 9)

    def work():
        a = bcjr_mod.apply_rht_gpu(W, sl, sr)
        b = bcjr_mod.apply_inverse_rht_batched(Wb, slb, srb)
        c = ops.dequant(spec, start, cb._bcjr_lut, m, n, 16, 16, 0.03, packed=packed)
        return a, b, bcjr_mod.apply_inverse_rht_gpu(c, sl, sr)

    ref = [t.clone() for t in work()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for _ in range(2):
            work()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = work()
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for o, r in zip(outs, ref):
            assert torch.equal(o, r)
        _ = torch.randn(4096, device="cuda").sum().item()  # eager work between replays


def test_reference_named_viterbi_and_numpy_ste(bcjr_mod, oracle):
    """viterbi_encode_v_batched_cuda keeps the reference's fixed-shape contract
    (src/viterbi/cuda_kernel.py:166-220); quantize_forward_numpy
    (src/qat/ste.py:213-267) against the same steps on the oracle, bit for bit
    (m*n an even power of two, numpy float32 RMS as the reference computes it)."""
    _say("reference-named viterbi + numpy STE")
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
    cb = bcjr_mod.make_hyb_codebook_gpu(lut, 9, 16, "cuda")
    x = torch.randn(8, 256, device="cuda")
    a = bcjr_mod.viterbi_encode_v_batched_cuda(x, cb)
    b = bcjr_mod.viterbi_encode_v_batched_hip(x, cb, L=16, k=2, V=2)
    assert all(torch.equal(p, q) for p, q in zip(a, b))
    with pytest.raises(AssertionError):
        bcjr_mod.viterbi_encode_v_batched_cuda(x, torch.zeros(4096, 2, device="cuda"))
    with pytest.raises(AssertionError):
        bcjr_mod.viterbi_encode_v_batched_cuda(x[:, :255], cb)

    m, n = 64, 256
    rng = np.random.default_rng(17)
    W = (rng.standard_normal((m, n)) * 0.03).astype(np.float32)
    sl, sr = _signs(m, 31), _signs(n, 32)
    W_q, W_scale, walks, bits, start = bcjr_mod.quantize_forward_numpy(W, sl, sr, cb)
    Wt = oracle.rht(W, sl, sr)
    scale = float(np.sqrt((Wt ** 2).mean()))
    assert W_scale == scale
    seqs, info = tile_for_viterbi(torch.tensor(Wt / scale), 16, 16)
    walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(seqs.numpy().reshape(seqs.shape[0], -1, 2), cb.cpu().numpy(),
                                                          16, 4)
    assert (bits == bits_r).all() and (start == start_r).all()
    assert (walks == walk_r.astype(np.int64)).all()
    Wtq = untile_from_viterbi(torch.tensor(recon_r.reshape(seqs.shape[0], -1)), info, (m, n), 16, 16).numpy() * scale
    assert np.array_equal(W_q, oracle.inverse_rht(Wtq.astype(np.float32), sl, sr))
