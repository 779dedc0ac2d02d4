"""GPU parity of the constrained and tail-biting Viterbi (bcjr_viterbi_constrained
through the C ABI) and of the numpy-facing API of src/viterbi/encode.py.

Bit-exact against the oracle (walk, bitstream, start, recon; mse to 1e-6): the
constrained encoder of encode.py:328-389 (pinned on the CPU by brute force over
the paths meeting the constraint), Algorithm 4 tail-biting (encode.py:392-422)
and the reference's own tail-biting gates at L=16 (test_viterbi.py:135-197,
test_viterbi_v2.py:98-147); the return_trace=True lattices (bcjr_viterbi_trace)
bit-exact against the oracle's restatement of encode.py:250-307, including the
reference's own trace gate shape (test_viterbi_cuda_forward.py:25-80)."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _codebook(bcjr, kind, L, rng):
    if kind == "1mad":
        cb = bcjr.make_1mad_codebook(L, "cuda")
    elif kind == "3inst":
        cb = bcjr.make_3inst_codebook(L, "cuda")
    elif kind == "hyb":
        lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
        cb = bcjr.make_hyb_codebook_gpu(lut, Q=9, L_bits=L, device="cuda")
    elif kind == "table":
        cb = torch.tensor(rng.standard_normal((1 << L, 1)).astype(np.float32), device="cuda")
    else:
        raise ValueError(kind)
    return cb, cb.cpu().numpy()


def _same(got, ref, B, N, V):
    bits, start, recon, mse, out = got
    walk_r, bits_r, start_r, recon_r, mse_r = ref[:5]
    assert np.array_equal(out["walk"].cpu().numpy(), walk_r)
    assert np.array_equal(bits.cpu().numpy(), bits_r)
    assert np.array_equal(start.cpu().numpy(), start_r)
    assert np.array_equal(recon.cpu().numpy(), recon_r.reshape(B, N * V))
    assert np.abs(mse.cpu().numpy() - mse_r).max() < 1e-6


# (L, k, V, N, B, codebook, overlap_bits or None for L - kV)
CONS = [
    (12, 2, 1, 256, 6, "1mad", None),
    (12, 2, 2, 128, 4, "hyb", None),
    (12, 2, 1, 64, 4, "table", 5),
    (14, 2, 1, 128, 3, "3inst", None),   # 1024-thread instance
    (16, 2, 1, 256, 3, "3inst", None),
    (16, 2, 2, 128, 2, "hyb", None),     # 1024 threads, LUT copies
]


@pytest.mark.parametrize("L,k,V,N,B,kind,ob", CONS)
def test_constrained_bit_exact(bcjr_mod, oracle, L, k, V, N, B, kind, ob):
    _say(f"constrained L={L} k={k} V={V} N={N} B={B} {kind} ob={ob}")
    rng = np.random.default_rng(L * 3 + N)
    cb, cb_np = _codebook(bcjr_mod, kind, L, rng)
    kV = k * V
    obits = L - kV if ob is None else ob
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    ov = rng.integers(0, 1 << obits, B).astype(np.int32)
    got = bcjr_mod.viterbi_encode_constrained_v_batched_hip(
        torch.tensor(seq.reshape(B, N * V), device="cuda"), cb, torch.tensor(ov, device="cuda"), ob,
        L=L, k=k, V=V, return_all=True)
    ref = oracle.viterbi(seq, cb_np, L, kV, overlap=ov, overlap_bits=obits)
    _same(got, ref, B, N, V)
    walk = got[4]["walk"].cpu().numpy()
    assert np.array_equal(walk[:, 0] >> (L - obits), ov)
    assert np.array_equal(walk[:, -1] & ((1 << obits) - 1), ov)


def test_constrained_infeasible_flags_start(bcjr_mod, oracle):
    """One step, overlap L - kV: first and last state coincide, so only values
    whose two windows agree have a walk; the others get start = -1, as the
    oracle (which the brute force pins) reports."""
    _say("constrained infeasible")
    L, k, V = 8, 2, 1
    rng = np.random.default_rng(5)
    cb, cb_np = _codebook(bcjr_mod, "table", L, rng)
    ov = np.arange(1 << (L - 2), dtype=np.int32)
    seq = np.repeat(rng.standard_normal((1, 1, 1)).astype(np.float32), len(ov), 0)
    bits, start, recon, mse = bcjr_mod.viterbi_encode_constrained_v_batched_hip(
        torch.tensor(seq.reshape(len(ov), 1), device="cuda"), cb, torch.tensor(ov, device="cuda"),
        L=L, k=k, V=V)
    ref_start = oracle.viterbi(seq, cb_np, L, 2, overlap=ov, overlap_bits=L - 2)[2]
    assert np.array_equal(start.cpu().numpy(), ref_start)
    assert (ref_start == -1).any() and (ref_start >= 0).any()


@pytest.mark.parametrize("L,k,V,N,B,kind", [(12, 2, 1, 256, 6, "1mad"), (16, 2, 1, 256, 4, "3inst"),
                                            (16, 2, 2, 128, 3, "hyb"), (10, 1, 1, 101, 3, "table")])
def test_tailbiting_bit_exact(bcjr_mod, oracle, L, k, V, N, B, kind):
    _say(f"tail-biting L={L} k={k} V={V} N={N} B={B} {kind}")
    rng = np.random.default_rng(L + N)
    cb, cb_np = _codebook(bcjr_mod, kind, L, rng)
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    bits, start, recon, mse, ov, out = bcjr_mod.viterbi_encode_tailbiting_v_batched_hip(
        torch.tensor(seq.reshape(B, N * V), device="cuda"), cb, L=L, k=k, V=V, return_all=True)
    ref = oracle.viterbi_tailbiting(seq, cb_np, L, k, V)
    assert np.array_equal(ov.cpu().numpy(), ref[5])
    _same((bits, start, recon, mse, out), ref, B, N, V)


@pytest.mark.parametrize("V,kind,gap", [(1, "1mad", 0.005), (2, "hyb", 0.006)])
def test_tailbiting_reference_gate(bcjr_mod, V, kind, gap):
    """test_viterbi.py:135-197 (V=1, 1MAD, 32 sequences) and
    test_viterbi_v2.py:98-147 (V=2, HYB, 16 sequences; a random 2^9 x 2 LUT
    stands in for the reference's k-means LUT file, which the repository does not
    ship): every walk wraps around (s_0 >> kV == s_{N-1} mod 2^(L-kV) ==
    overlap) and the mean MSE is within the gate of the unconstrained one."""
    _say(f"tail-biting gate V={V} {kind}")
    L, k, T = 16, 2, 256
    rng = np.random.default_rng(42)
    cb, _ = _codebook(bcjr_mod, kind, L, rng)
    B = 32 if V == 1 else 16
    x = torch.tensor(rng.standard_normal((B, T)).astype(np.float32), device="cuda")
    _, _, _, mse0 = bcjr_mod.viterbi_encode_v_batched_hip(x, cb, L=L, k=k, V=V)
    bits, start, recon, mse, ov, out = bcjr_mod.viterbi_encode_tailbiting_v_batched_hip(
        x, cb, L=L, k=k, V=V, return_all=True)
    kV = k * V
    walk = out["walk"].cpu().numpy()
    ov = ov.cpu().numpy()
    assert (start.cpu().numpy() >= 0).all()
    assert np.array_equal(walk[:, 0] >> kV, ov)
    assert np.array_equal(walk[:, -1] & ((1 << (L - kV)) - 1), ov)
    assert abs(float(mse.mean()) - float(mse0.mean())) < gap


def test_numpy_api_matches_oracle(bcjr_mod, oracle):
    """The reference-named functions of src/viterbi/encode.py with a decode_fn:
    single-sequence, V=2, batched, decode, constrained and tail-biting, against
    the oracle; mse as the reference forms it from recon."""
    _say("numpy encode API")
    from bcjr import encode as E
    rng = np.random.default_rng(17)
    L, k = 12, 2
    cb1 = oracle.codebook(oracle.CODE_1MAD, L)[:, 0]
    dec1 = lambda s: cb1[s.astype(np.int64)]  # noqa: E731
    seq = rng.standard_normal(128).astype(np.float32)
    bs, st, rc, mse = E.viterbi_encode(seq, L, k, dec1)
    w_r, b_r, s_r, r_r, _ = oracle.viterbi(seq[None, :, None], cb1[:, None], L, k)
    assert bs.dtype == np.int32 and np.array_equal(bs, b_r[0]) and st == int(s_r[0])
    assert np.array_equal(rc, r_r[0, :, 0]) and mse == float(np.mean((rc - seq) ** 2))
    assert np.array_equal(E.viterbi_decode(bs, st, L, k, dec1), rc)

    cb2 = rng.standard_normal((1 << L, 2)).astype(np.float32)
    dec2 = lambda s: cb2[s.astype(np.int64)]  # noqa: E731
    seq2 = rng.standard_normal(96).astype(np.float32)
    bs, st, rc, mse = E.viterbi_encode_v(seq2, L, k, 2, dec2)
    w_r, b_r, s_r, r_r, _ = oracle.viterbi(seq2.reshape(1, 48, 2), cb2, L, 4)
    assert np.array_equal(bs, b_r[0]) and st == int(s_r[0]) and np.array_equal(rc, r_r.reshape(-1))
    assert np.array_equal(E.viterbi_decode_v(bs, st, L, k, 2, dec2), rc)

    seqs = rng.standard_normal((5, 96)).astype(np.float32)
    bb, ss, rr, mm = E.viterbi_encode_v_batched(seqs, L, k, 2, dec2)
    for i in range(5):
        b1, s1, r1, m1 = E.viterbi_encode_v(seqs[i], L, k, 2, dec2)
        assert np.array_equal(bb[i], b1) and ss[i] == s1 and np.array_equal(rr[i], r1)
        assert abs(float(mm[i]) - m1) < 1e-7

    bs, st, rc, mse, ov = E.viterbi_encode_tailbiting(seq, L, k, dec1)
    ref = oracle.viterbi_tailbiting(seq[None, :, None], cb1[:, None], L, k, 1)
    assert ov == int(ref[5][0]) and np.array_equal(bs, ref[1][0]) and st == int(ref[2][0])
    b2, s2, r2, m2 = E.viterbi_encode_constrained(seq, L, k, dec1, L - k, ov)
    assert np.array_equal(b2, bs) and s2 == st and np.array_equal(r2, rc) and m2 == mse
    bs, st, rc, mse, ov = E.viterbi_encode_tailbiting_v(seq2, L, k, 2, dec2)
    ref = oracle.viterbi_tailbiting(seq2.reshape(1, 48, 2), cb2, L, k, 2)
    assert ov == int(ref[5][0]) and np.array_equal(bs, ref[1][0])

    # one step with a value whose two windows disagree: no walk, as the reference raises
    with pytest.raises(RuntimeError, match="No valid tail-biting walk"):
        E.viterbi_encode_constrained(seq[:1], L, k, dec1, L - k, 1)


# (L, k, V, N, B, codebook) straight through ops.viterbi_trace
TRACE = [
    (6, 1, 1, 9, 3, "table"),     # kV = 1
    (10, 2, 1, 40, 3, "1mad"),
    (12, 2, 2, 24, 2, "hyb"),     # kV = 4
    (8, 4, 1, 7, 2, "table"),     # kV = 4, V = 1
    (16, 2, 1, 6, 2, "3inst"),    # 16 reduced indices per thread
]


@pytest.mark.parametrize("L,k,V,N,B,kind", TRACE)
def test_viterbi_trace_bit_exact(bcjr_mod, oracle, L, k, V, N, B, kind):
    _say(f"viterbi trace L={L} k={k} V={V} N={N} B={B} {kind}")
    from bcjr import ops
    rng = np.random.default_rng(L + 7 * N)
    if kind == "hyb":
        cb, cb_np = _codebook(bcjr_mod, kind, L, rng)
    else:
        cb_np = (oracle.codebook({"1mad": oracle.CODE_1MAD, "3inst": oracle.CODE_3INST}[kind], L) if kind != "table"
                 else rng.standard_normal((1 << L, V)).astype(np.float32))
        cb = torch.tensor(cb_np, device="cuda")
    seq = rng.standard_normal((B, N, V)).astype(np.float32)
    trace, bp = ops.viterbi_trace(ops.Spec(L, k, V, ops.CODE_TABLE), torch.tensor(seq, device="cuda"), cb)
    trace, bp = trace.cpu().numpy(), bp.cpu().numpy()
    for b in range(B):
        t_r, b_r = oracle.viterbi_trace(seq[b], cb_np, L, k * V)
        assert np.array_equal(trace[b], t_r), b
        assert np.array_equal(bp[b], b_r), b


def test_return_trace_api_and_reference_gate_shape(bcjr_mod, oracle):
    """viterbi_encode / viterbi_encode_v with return_trace=True: the four usual
    outputs unchanged, plus trace_err and backpointers bit-exact against the
    oracle; at the reference's trace gate shape (L=16, k=2, V=2, HYB decoder,
    256 weights) the final row is the cum_err that gate compares."""
    _say("return_trace API")
    from bcjr import encode as E
    rng = np.random.default_rng(23)
    L, k = 12, 2
    cb1 = oracle.codebook(oracle.CODE_1MAD, L)[:, 0]
    dec1 = lambda s: cb1[s.astype(np.int64)]  # noqa: E731
    seq = rng.standard_normal(64).astype(np.float32)
    out = E.viterbi_encode(seq, L, k, dec1, return_trace=True)
    plain = E.viterbi_encode(seq, L, k, dec1)
    assert len(out) == 6 and np.array_equal(out[0], plain[0]) and out[1] == plain[1]
    assert np.array_equal(out[2], plain[2]) and out[3] == plain[3]
    t_r, b_r = oracle.viterbi_trace(seq[:, None], cb1[:, None], L, k)
    assert out[4].shape == (64, 1 << L) and out[4].dtype == np.float32 and out[5].dtype == np.int32
    assert np.array_equal(out[4], t_r) and np.array_equal(out[5], b_r)
    # backtrace through the returned backpointers gives the returned walk
    w = [int(np.argmin(out[4][-1]))]
    for t in range(63, 0, -1):
        w.append(int(out[5][t, w[-1]]))
    assert (np.array(w[::-1]) & 3).tolist() == out[0].tolist() and int(out[5][0, w[-1]]) == out[1]

    lut = np.random.default_rng(2).standard_normal((512, 2)).astype(np.float32)
    cbh = bcjr_mod.make_hyb_codebook_gpu(lut, Q=9, L_bits=16, device="cuda").cpu().numpy()
    dech = lambda s: cbh[s.astype(np.int64)]  # noqa: E731
    seq2 = rng.standard_normal(256).astype(np.float32)
    out = E.viterbi_encode_v(seq2, 16, 2, 2, dech, return_trace=True)
    t_r, b_r = oracle.viterbi_trace(seq2.reshape(128, 2), cbh, 16, 4)
    assert np.array_equal(out[4], t_r) and np.array_equal(out[5], b_r)
    assert int(np.argmin(out[4][-1])) == int(np.argmin(t_r[-1]))
