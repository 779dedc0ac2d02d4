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


def _rht_cases(n=40, seed=7):
    """(E, m, n): the extremes of the supported range, then powers of two with
    m*n <= 2^22, each batched E = 1..3 times."""
    rng = np.random.default_rng(seed)
    out = [(1, 1, 1), (1, 1, 16384), (2, 16384, 1), (1, 2, 8192), (1, 4096, 1024)]
    while len(out) < n:
        lm, ln = int(rng.integers(0, 15)), int(rng.integers(0, 15))
        if lm + ln <= 22:
            out.append((int(rng.integers(1, 4)), 1 << lm, 1 << ln))
    return out


@pytest.mark.parametrize("E,m,n", _rht_cases())
def test_rht_sweep_vs_oracle(bcjr_mod, oracle, E, m, n):
    """Forward and inverse RHT, batched and single, against the oracle's float32
    butterflies: bit-exact when m*n is an even power of two (the scale 1/sqrt(mn)
    is exact), within 2 ulp of the largest value otherwise."""
    print(f"rht sweep E={E} {m}x{n}", flush=True)
    rng = np.random.default_rng(E * 100003 + m * 31 + n)
    W = _weights(rng, (E, m, n), tails=bool(m & 1))
    SL = rng.choice([-1.0, 1.0], size=(E, m)).astype(np.float32)
    SR = rng.choice([-1.0, 1.0], size=(E, n)).astype(np.float32)
    Wd, sl, sr = (torch.tensor(a, device="cuda") for a in (W, SL, SR))
    Wt = bcjr_mod.apply_rht_batched(Wd, sl, sr)
    back = bcjr_mod.apply_inverse_rht_batched(Wt, sl, sr)
    exact = ((m * n).bit_length() - 1) % 2 == 0
    for e in range(E):
        ref = oracle.rht(W[e], SL[e], SR[e])
        ref_back = oracle.inverse_rht(Wt[e].cpu().numpy(), SL[e], SR[e])
        got, got_back = Wt[e].cpu().numpy(), back[e].cpu().numpy()
        if exact:
            assert np.array_equal(got, ref)
            assert np.array_equal(got_back, ref_back)
        else:
            assert np.abs(got - ref).max() <= 2 * np.spacing(np.abs(ref).max())
            assert np.abs(got_back - ref_back).max() <= 2 * np.spacing(np.abs(ref_back).max())
        assert torch.equal(Wt[e], bcjr_mod.apply_rht_gpu(Wd[e], sl[e], sr[e]))


def _dequant_cases(n=32, seed=11):
    """(L, k, V, kind, Tx, Ty, m, n): tiles of any shape holding whole steps,
    matrices of 1..6 x 1..6 tiles."""
    rng = np.random.default_rng(seed)
    out = [(16, 2, 2, "hyb", 16, 16, 64, 256), (16, 2, 1, "3inst", 16, 16, 32, 64)]
    while len(out) < n:
        k, V = SHAPES[int(rng.integers(len(SHAPES)))]
        kV = k * V
        L = int(rng.integers(2 * kV, (11 if kV == 1 else 16) + 1))
        kinds = ["table"] + (["1mad", "3inst"] if V == 1 else ["hyb"])
        kind = kinds[int(rng.integers(len(kinds)))]
        Tx, Ty = int(rng.choice([1, 2, 4, 8, 16, 3, 6])), int(rng.choice([1, 2, 4, 8, 16, 12, 5]))
        if (Tx * Ty) % V:
            continue
        out.append((L, k, V, kind, Tx, Ty, Tx * int(rng.integers(1, 7)), Ty * int(rng.integers(1, 7))))
    return out


@pytest.mark.parametrize("L,k,V,kind,Tx,Ty,m,n", _dequant_cases())
def test_dequant_sweep_vs_oracle(bcjr_mod, oracle, L, k, V, kind, Tx, Ty, m, n):
    """The rotated-basis dequantization fl32(W_scale * c(walk)) from uint8 and
    (where k*V divides 8) packed bitstreams, bit-exact against the oracle."""
    from bcjr.serialize import dequant_target_gpu, pack_bitstreams
    print(f"dequant sweep L={L} k={k} V={V} {kind} tiles {Tx}x{Ty} of {m}x{n}", flush=True)
    rng = np.random.default_rng(L * 7919 + Tx * 131 + Ty * 17 + m + n)
    cb, cb_np = _codebook(bcjr_mod, kind, L, V, rng)
    kV = k * V
    nc, nr, N = n // Ty, m // Tx, Tx * Ty // V
    p = {
        "bitstreams": rng.integers(0, 1 << kV, (nc, nr, N)).astype(np.uint8),
        "start_states": rng.integers(0, 1 << L, (nc, nr)).astype(np.int32),
        "sign_l": np.sign(rng.standard_normal(m)).astype(np.int8),
        "sign_r": np.sign(rng.standard_normal(n)).astype(np.int8),
        "W_scale": float(rng.uniform(0.005, 0.05)),
        "shape": (m, n),
        "config": {"L": L, "k": k, "V": V, "Tx": Tx, "Ty": Ty},
    }
    ref = (oracle.dequant_unit(p["bitstreams"], p["start_states"], cb_np, (m, n), L, kV, Tx, Ty)
           * p["W_scale"]).astype(np.float32)
    got = dequant_target_gpu(p, rotated=True, codebook=cb)
    assert np.array_equal(got.cpu().numpy(), ref)
    if 8 % kV == 0:
        pk = {kk: v for kk, v in p.items() if kk != "bitstreams"}
        pk["packed"] = pack_bitstreams(p["bitstreams"], kV)
        pk["n_steps"] = N
        assert torch.equal(dequant_target_gpu(pk, rotated=True, codebook=cb), got)


def _viterbi_cases(n=24, seed=13):
    """(L, k, V, kind, N, B, overlap_bits): the constrained encoder over random
    shapes, overlap windows from 0 bits (unconstrained) to L - kV (tail-biting)."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k, V = SHAPES[int(rng.integers(len(SHAPES)))]
        kV = k * V
        L = int(rng.integers(2 * kV, (11 if kV == 1 else 16) + 1))
        kinds = ["table"] + (["1mad", "3inst"] if V == 1 else ["hyb"])
        kind = kinds[int(rng.integers(len(kinds)))]
        N = int(rng.choice(LENGTHS))
        B = int(rng.integers(1, 9))
        out.append((L, k, V, kind, N, B, int(rng.integers(0, L - kV + 1))))
    return out


@pytest.mark.parametrize("L,k,V,kind,N,B,ob", _viterbi_cases())
def test_constrained_viterbi_sweep_vs_oracle(bcjr_mod, oracle, L, k, V, kind, N, B, ob):
    """Walk, bitstream, start state (-1 where no walk meets the constraint) and
    reconstruction bit-exact against the oracle's constrained encoder."""
    print(f"constrained sweep L={L} k={k} V={V} {kind} N={N} B={B} ob={ob}", flush=True)
    rng = np.random.default_rng(L * 613 + N * 7 + B + ob)
    cb, cb_np = _codebook(bcjr_mod, kind, L, V, rng)
    seq = _weights(rng, (B, N, V), tails=bool(N & 1))
    ov = rng.integers(0, 1 << ob, B).astype(np.int32)
    bits, start, recon, mse, out = bcjr_mod.viterbi_encode_constrained_v_batched_hip(
        torch.tensor(seq.reshape(B, N * V), device="cuda"), cb, torch.tensor(ov, device="cuda"), ob,
        L=L, k=k, V=V, return_all=True)
    walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(seq, cb_np, L, k * V, overlap=ov, overlap_bits=ob)
    assert np.array_equal(start.cpu().numpy(), start_r)
    ok = start_r >= 0  # the other sequences' walks are unspecified
    assert np.array_equal(out["walk"].cpu().numpy()[ok], walk_r[ok])
    assert np.array_equal(bits.cpu().numpy()[ok], bits_r[ok])
    assert np.array_equal(recon.cpu().numpy()[ok], recon_r.reshape(B, N * V)[ok])


def _weight_cases(n=12, seed=17):
    """(m, n, L, k, V, kind, T): one weight through bcjr_quantize_weight, shapes
    of 1..32 16x16 tiles (powers of two for the RHT)."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        m, nn = 1 << int(rng.integers(4, 10)), 1 << int(rng.integers(4, 10))
        if m * nn > 8192:
            continue
        k, V = [(2, 1), (1, 2), (2, 2), (1, 1)][int(rng.integers(4))]
        kV = k * V
        L = int(rng.integers(max(2 * kV, 6), 13))
        kinds = ["table"] + (["1mad", "3inst"] if V == 1 else ["hyb"])
        kind = kinds[int(rng.integers(len(kinds)))]
        T = round(float(np.exp(rng.uniform(np.log(0.05), np.log(1.0)))), 4)
        out.append((m, nn, L, k, V, kind, T))
    return out


@pytest.mark.parametrize("m,n,L,k,V,kind,T", _weight_cases())
def test_quantize_weight_sweep_vs_oracle(bcjr_mod, oracle, m, n, L, k, V, kind, T):
    """bcjr_quantize_weight (RHT, RMS scale, 16x16 tiles, BCJR, back) and its
    gradient against the same composition on the oracle."""
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    print(f"quantize_weight sweep {m}x{n} L={L} k={k} V={V} {kind} T={T}", flush=True)
    rng = np.random.default_rng(m * 131 + n * 7 + L)
    cb, cb_np = _codebook(bcjr_mod, kind, L, V, rng)
    W = (rng.standard_normal((m, n)) * 0.02).astype(np.float32)
    g = rng.standard_normal((m, n)).astype(np.float32)
    sl = rng.choice([-1.0, 1.0], size=m).astype(np.float32)
    sr = rng.choice([-1.0, 1.0], size=n).astype(np.float32)
    Wd = torch.tensor(W, device="cuda", requires_grad=True)
    Wq = bcjr_mod.bcjr_quantize_weight(Wd, torch.tensor(sl, device="cuda"), torch.tensor(sr, device="cuda"),
                                       cb, T, L=L, k=k, V=V)
    (Wq * torch.tensor(g, device="cuda")).sum().backward()

    Wt = oracle.rht(W, sl, sr)
    scale = np.float32(np.sqrt((Wt ** 2).mean(dtype=np.float32)))
    seqs, info = tile_for_viterbi(torch.tensor(Wt / scale), 16, 16)
    seqs = seqs.numpy().reshape(seqs.shape[0], -1, V)
    soft, _ = oracle.bcjr_forward(seqs, cb_np, T, L, k * V)
    Wtq = untile_from_viterbi(torch.tensor(soft.reshape(seqs.shape[0], -1)), info, (m, n), 16, 16).numpy()
    ref = oracle.inverse_rht(Wtq * scale, sl, sr)
    assert np.abs(Wq.detach().cpu().numpy() - ref).max() <= SOFT_TOL * np.abs(ref).max()
    gt_tiles, _ = tile_for_viterbi(torch.tensor(oracle.rht(g, sl, sr) * scale), 16, 16)
    d_seq = oracle.bcjr_backward(seqs, cb_np, T, L, k * V, gt_tiles.numpy().reshape(seqs.shape))
    d_wt = untile_from_viterbi(torch.tensor(d_seq.reshape(seqs.shape[0], -1) / scale), info, (m, n), 16, 16).numpy()
    grad_ref = oracle.inverse_rht(d_wt, sl, sr)
    assert np.abs(Wd.grad.cpu().numpy() - grad_ref).max() <= GRAD_TOL * np.abs(grad_ref).max()


@pytest.mark.parametrize("seed", range(6))
def test_experts_sweep_vs_per_weight_loop(bcjr_mod, seed):
    """bcjr_quantize_experts over a random mixture of 2..7 weights of 1..4
    distinct shapes (repeated shapes share one batched RHT), a temperature per
    weight, against one bcjr_quantize_weight per weight: values and gradients."""
    rng = np.random.default_rng(500 + seed)
    palette = [(1 << int(rng.integers(4, 9)), 1 << int(rng.integers(4, 9))) for _ in range(int(rng.integers(1, 5)))]
    shapes = [palette[int(rng.integers(len(palette)))] for _ in range(int(rng.integers(2, 8)))]
    Ts = torch.tensor(np.exp(rng.uniform(np.log(0.05), np.log(0.5), len(shapes))).astype(np.float32), device="cuda")
    print(f"experts sweep seed={seed} shapes={shapes}", flush=True)
    cb = bcjr_mod.make_3inst_codebook(12, "cuda")
    Ws = [torch.tensor((rng.standard_normal(s) * 0.02).astype(np.float32), device="cuda") for s in shapes]
    sl = [torch.tensor(rng.choice([-1.0, 1.0], size=s[0]).astype(np.float32), device="cuda") for s in shapes]
    sr = [torch.tensor(rng.choice([-1.0, 1.0], size=s[1]).astype(np.float32), device="cuda") for s in shapes]
    Wd = [W.clone().requires_grad_(True) for W in Ws]
    outs = bcjr_mod.bcjr_quantize_experts(Wd, sl, sr, cb, Ts, L=12, k=2, V=1)
    gs = [torch.randn(s, device="cuda", generator=torch.Generator("cuda").manual_seed(seed)) for s in shapes]
    sum((o * g).sum() for o, g in zip(outs, gs)).backward()
    for e in range(len(shapes)):
        W1 = Ws[e].clone().requires_grad_(True)
        ref = bcjr_mod.bcjr_quantize_weight(W1, sl[e], sr[e], cb, Ts[e], L=12, k=2, V=1)
        (ref * gs[e]).sum().backward()
        assert (outs[e] - ref).abs().max() <= SOFT_TOL * ref.abs().max(), e
        assert (Wd[e].grad - W1.grad).abs().max() <= GRAD_TOL * W1.grad.abs().max(), e


def _ste_cases(n=12, seed=19):
    """(m, n, L, k, V, kind, packed): a weight through the hard quantizer, then
    stored, loaded and dequantized."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        m, nn = 1 << int(rng.integers(4, 10)), 1 << int(rng.integers(4, 10))
        if m * nn > 65536:
            continue
        k, V = [(2, 1), (1, 2), (2, 2), (1, 1)][int(rng.integers(4))]
        kV = k * V
        L = int(rng.integers(max(2 * kV, 6), (11 if kV == 1 else 16) + 1))
        kinds = ["table"] + (["1mad", "3inst"] if V == 1 else ["hyb"])
        out.append((m, nn, L, k, V, kinds[int(rng.integers(len(kinds)))], bool(rng.integers(2))))
    return out


@pytest.mark.parametrize("m,n,L,k,V,kind,packed", _ste_cases())
def test_ste_and_round_trip_sweep(bcjr_mod, oracle, m, n, L, k, V, kind, packed, tmp_path):
    """quantize_forward_gpu (RHT, RMS scale, tiles, Viterbi, back) against the
    oracle's Viterbi composed with the same steps (bit-exact where m*n is an even
    power of two, else within the inverse RHT's scale rounding), then save (uint8
    or packed file) -> load -> dequantize equal to it bit for bit."""
    import bcjr
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    print(f"ste sweep {m}x{n} L={L} k={k} V={V} {kind} packed={packed}", flush=True)
    rng = np.random.default_rng(m * 17 + n * 3 + L)
    cb, cb_np = _codebook(bcjr_mod, kind, L, V, rng)
    sl = torch.tensor(rng.choice([-1.0, 1.0], size=m).astype(np.float32), device="cuda")
    sr = torch.tensor(rng.choice([-1.0, 1.0], size=n).astype(np.float32), device="cuda")
    W = torch.tensor((rng.standard_normal((m, n)) * 0.03).astype(np.float32), device="cuda")
    Wq = bcjr.quantize_forward_gpu(W, sl, sr, cb, k=k)

    Wt = bcjr.apply_rht_gpu(W, sl, sr)
    s = Wt.pow(2).mean().sqrt().clamp(min=1e-30)
    seqs, info = tile_for_viterbi((Wt / s).cpu(), 16, 16)
    walk_r, bits_r, start_r, recon_r, _ = oracle.viterbi(seqs.numpy().reshape(seqs.shape[0], -1, V), cb_np, L, k * V)
    Wtq = untile_from_viterbi(torch.tensor(recon_r.reshape(seqs.shape[0], -1)), info, (m, n), 16, 16)
    ref = oracle.inverse_rht((Wtq * s.cpu()).numpy(), sl.cpu().numpy(), sr.cpu().numpy())
    if ((m * n).bit_length() - 1) % 2 == 0:  # 1/sqrt(mn) exact
        assert np.array_equal(Wq.cpu().numpy(), ref)
    else:
        assert np.abs(Wq.cpu().numpy() - ref).max() <= 2 * np.spacing(np.abs(ref).max())

    nr, nc = info
    args = dict(bitstreams=bits_r.reshape(nc, nr, -1).astype(np.uint8), start_states=start_r.reshape(nc, nr),
                sign_l=sl.cpu().numpy(), sign_r=sr.cpu().numpy(), W_scale=float(s), shape=(m, n),
                meta={"layer": 0, "kind": "mlp", "proj": kind},
                config={"L": L, "k": k, "V": V, "Tx": 16, "Ty": 16})
    if packed and 8 % (k * V) != 0:
        packed = False
    path = str(tmp_path / ("w.safetensors" if packed else "w.pt"))
    (bcjr.save_packed if packed else bcjr.save_quantized)(path, **args)
    assert torch.equal(bcjr.dequant_target_gpu(bcjr.load_quantized(path), codebook=cb), Wq)


def test_every_accepted_problem_has_a_launch_plan(bcjr_mod):
    """Every problem the C ABI's validation accepts (each built k*V and V, every
    L it allows, every code it allows there, HYB at Q = 9 and Q = 10, short and
    long sequences) gets a launch plan for the forward, the backward and the
    Viterbi: a kernel instance exists and is resident.  No kernel runs.  A
    generator code at k*V = 1 is refused by the validation itself."""
    import ctypes
    from bcjr import _lib as BL
    lib = bcjr_mod.load_library()
    missing = []
    for k, V in SHAPES:
        kV = k * V
        for L in range(2 * kV, (11 if kV == 1 else 16) + 1):
            codes = [(BL.CODE_TABLE, 9)]
            if kV > 1:  # k*V = 1 is built for the table code only
                codes += [(BL.CODE_1MAD, 9), (BL.CODE_3INST, 9)] if V == 1 else [(BL.CODE_HYB, 9), (BL.CODE_HYB, 10)]
            for code, Q in codes:
                for N in (1, 256):
                    for op in (BL.OP_FORWARD, BL.OP_BACKWARD, BL.OP_VITERBI):
                        p = BL.Problem(L, k, V, 4, N, code, Q, 0)
                        n = ctypes.c_size_t(0)
                        if lib.bcjr_workspace_bytes(ctypes.byref(p), op, ctypes.byref(n)) != 0 or n.value == 0:
                            missing.append((L, k, V, code, Q, N, op, lib.bcjr_last_error().decode()))
    assert not missing, "\n".join(map(str, missing[:40]))
    p = BL.Problem(8, 1, 1, 4, 16, BL.CODE_3INST, 9, 0)
    assert lib.bcjr_workspace_bytes(ctypes.byref(p), BL.OP_FORWARD, ctypes.byref(ctypes.c_size_t(0))) == \
        BL.BCJR_EUNSUPPORTED
    assert "table code only" in lib.bcjr_last_error().decode()


def _diag_cases(n=16, seed=23):
    """(L, k, V, kind, N, B, T): small trellises for the diagnostics outputs."""
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n:
        k, V = SHAPES[int(rng.integers(len(SHAPES)))]
        kV = k * V
        L = int(rng.integers(2 * kV, 13))
        kinds = ["table"] + (["1mad", "3inst"] if V == 1 else ["hyb"])
        kind = kinds[int(rng.integers(len(kinds)))]
        N = int(rng.choice([1, 2, 5, 16, 33, 48]))
        T = round(float(np.exp(rng.uniform(np.log(0.1), np.log(1.5)))), 4)
        out.append((L, k, V, kind, N, int(rng.integers(1, 4)), T))
    return out


@pytest.mark.parametrize("L,k,V,kind,N,B,T", _diag_cases())
def test_diagnostics_sweep_vs_oracle(bcjr_mod, oracle, L, k, V, kind, N, B, T):
    """return_internals (P, log alpha, log beta per state) against the gather
    form of forward_backward.py; the marginal entropy against the oracle; the
    walk replay from bitstreams and from packed bytes, and the Viterbi trace,
    bit-exact."""
    from bcjr import bcjr_forward_backward, viterbi_decode_v_batched, viterbi_encode_v_batched_hip, ops
    print(f"diagnostics sweep L={L} k={k} V={V} {kind} N={N} B={B} T={T}", flush=True)
    rng = np.random.default_rng(L * 389 + N * 11 + B)
    cb, cb_np = _codebook(bcjr_mod, kind, L, V, rng)
    seq = _weights(rng, (B, N, V), tails=False)
    x = torch.tensor(seq, device="cuda")
    soft, logZ, P, la, lb = bcjr_forward_backward(x, cb, T, L=L, k=k, V=V, return_internals=True)
    s2, z2, P2, la2, lb2 = oracle.naive_forward(seq, cb_np, T, L, k * V, return_internals=True)
    assert max_rel(soft.detach().cpu().numpy(), s2) < SOFT_TOL
    assert np.abs(P.cpu().numpy() - P2).max() < 1e-5
    assert np.abs(la.cpu().numpy() - la2).max() < 1e-4 * max(1.0, np.abs(la2).max())
    assert np.abs(lb.cpu().numpy() - lb2).max() < 1e-4 * max(1.0, np.abs(lb2).max())
    H = bcjr_mod.bcjr_marginal_entropy(x, cb, T, L=L, k=k, V=V).cpu().numpy().astype(np.float64)
    H_ref = oracle.marginal_entropy(seq, cb_np, T, L, k * V)
    assert np.abs(H - H_ref).max() <= 1e-4 * max(1.0, float(np.abs(H_ref).max()))

    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(x.reshape(B, N * V), cb, L=L, k=k, V=V,
                                                                return_all=True)
    w1, r1 = viterbi_decode_v_batched(bits, start, cb, L=L, k=k, V=V)
    assert torch.equal(w1, out["walk"]) and torch.equal(r1, recon)
    if out["packed"] is not None:
        w2, r2 = viterbi_decode_v_batched(None, start, cb, L=L, k=k, V=V, packed=out["packed"], N=N)
        assert torch.equal(w2, out["walk"]) and torch.equal(r2, recon)
    tr, bp = ops.viterbi_trace(ops.Spec(L, k, V, ops.CODE_TABLE), x, cb)
    for b in range(B):
        t_r, b_r = oracle.viterbi_trace(seq[b], cb_np, L, k * V)
        assert np.array_equal(tr[b].cpu().numpy(), t_r)
        assert np.array_equal(bp[b].cpu().numpy(), b_r)


def test_calls_on_two_streams_overlap_safely(bcjr_mod):
    """Forward, backward and Viterbi of two independent batches issued on two
    streams (default priority) at once, each with its own workspace from the
    caching allocator of its stream: every output equals the same call made
    alone, bit for bit."""
    from bcjr import ops
    cb = bcjr_mod.make_3inst_codebook(14, "cuda")
    spec, table = bcjr_mod.codes.resolve_codebook(cb, 14, 2, 1, torch.device("cuda"))
    gen = torch.Generator("cuda").manual_seed(5)
    xs = [torch.randn(600, 64, 1, device="cuda", generator=gen) for _ in range(2)]
    gs = [torch.randn(600, 64, 1, device="cuda", generator=gen) for _ in range(2)]
    Ts = [0.1, 0.3]
    alone = []
    for x, g, T in zip(xs, gs, Ts):
        soft, logZ = ops.forward(spec, x, T, table)
        d = ops.backward(spec, x, T, table, g)
        v = ops.viterbi(spec, x, table)
        alone.append((soft, logZ, d, v["walk"], v["recon"]))
    torch.cuda.synchronize()
    streams = [torch.cuda.Stream(), torch.cuda.Stream()]
    for s in streams:
        s.wait_stream(torch.cuda.current_stream())
    both = [None, None]
    for _ in range(2):
        for i, s in enumerate(streams):
            with torch.cuda.stream(s):
                soft, logZ = ops.forward(spec, xs[i], Ts[i], table)
                d = ops.backward(spec, xs[i], Ts[i], table, gs[i])
                v = ops.viterbi(spec, xs[i], table)
                both[i] = (soft, logZ, d, v["walk"], v["recon"])
        torch.cuda.synchronize()
        for i in range(2):
            for got, ref in zip(both[i], alone[i]):
                assert torch.equal(got, ref)


def _max_N(lib, BL, L, k, V, code, op):
    """Longest sequence the launch plan accepts (LDS-bound), by bisection."""
    import ctypes
    lo, hi = 1, 4096
    def ok(N):
        p = BL.Problem(L, k, V, 1, N, code, 9, 0)
        return lib.bcjr_workspace_bytes(ctypes.byref(p), op, ctypes.byref(ctypes.c_size_t(0))) == 0
    assert ok(lo)
    if ok(hi):
        return hi
    while hi - lo > 1:
        mid = (lo + hi) // 2
        lo, hi = (mid, hi) if ok(mid) else (lo, mid)
    return lo


@pytest.mark.parametrize("L,k,V,kind", [(16, 2, 2, "hyb"), (16, 2, 2, "table"), (16, 1, 2, "hyb"),
                                        (11, 1, 1, "table"), (12, 2, 1, "1mad"), (16, 4, 1, "3inst")])
def test_longest_sequence_per_shape_vs_oracle(bcjr_mod, oracle, L, k, V, kind):
    """At each shape's longest accepted sequence (the LDS bound of its launch
    plan, or N = 4096): forward, gradient and Viterbi against the oracle, and
    one step more refused before any launch."""
    from bcjr import _lib as BL, bcjr_forward_backward, ops, viterbi_encode_v_batched_hip
    lib = bcjr_mod.load_library()
    rng = np.random.default_rng(L * 31 + k * 7 + V)
    cb, cb_np = _codebook(bcjr_mod, kind, L, V, rng)
    spec, table = bcjr_mod.codes.resolve_codebook(cb, L, k, V, torch.device("cuda"))
    limits = {op: _max_N(lib, BL, L, k, V, spec.code, op) for op in (BL.OP_FORWARD, BL.OP_BACKWARD, BL.OP_VITERBI)}
    print(f"longest L={L} k={k} V={V} {kind}: forward, backward, Viterbi {list(limits.values())}", flush=True)
    # N = 4096 is the ABI's own cap, not an LDS bound: a shorter sequence keeps the oracle quick there
    Nf, Nb, Nv = (n if n < 4096 else 1024 for n in limits.values())
    T = 0.2
    N = min(Nf, Nb)
    seq = rng.standard_normal((1, N, V)).astype(np.float32)
    g = rng.standard_normal((1, N, V)).astype(np.float32)
    x = torch.tensor(seq, device="cuda", requires_grad=True)
    soft, logZ = bcjr_forward_backward(x, cb, T, L=L, k=k, V=V)
    (soft * torch.tensor(g, device="cuda")).sum().backward()
    s_ref, z_ref = oracle.bcjr_forward(seq, cb_np, T, L, k * V)
    assert max_rel(soft.detach().cpu().numpy(), s_ref) < SOFT_TOL
    assert max_rel(x.grad.cpu().numpy(), oracle.bcjr_backward(seq, cb_np, T, L, k * V, g)) < GRAD_TOL
    if Nf > N:
        seq_f = rng.standard_normal((1, Nf, V)).astype(np.float32)
        soft_f, _ = ops.forward(spec, torch.tensor(seq_f, device="cuda"), T, table)
        assert max_rel(soft_f.cpu().numpy(), oracle.bcjr_forward(seq_f, cb_np, T, L, k * V)[0]) < SOFT_TOL
    seq_v = rng.standard_normal((1, Nv, V)).astype(np.float32)
    bits, start, recon, mse, out = viterbi_encode_v_batched_hip(torch.tensor(seq_v.reshape(1, -1), device="cuda"),
                                                                cb, L=L, k=k, V=V, return_all=True)
    assert np.array_equal(out["walk"].cpu().numpy(), oracle.viterbi(seq_v, cb_np, L, k * V)[0])
    for op, N_over in limits.items():
        if N_over < 4096:  # an LDS bound
            import ctypes
            p = BL.Problem(L, k, V, 1, N_over + 1, spec.code, 9, 0)
            assert lib.bcjr_workspace_bytes(ctypes.byref(p), op, ctypes.byref(ctypes.c_size_t(0))) == \
                BL.BCJR_EUNSUPPORTED
            assert "LDS" in lib.bcjr_last_error().decode()

