"""GPU parity of the on-disk format path: bcjr_dequant (walk replay + codebook +
untiling + scale in one kernel) and dequant_target (then the inverse RHT)
against the oracle restatement of src/quantize/serialize.py:56-107, walks
against src/quantize/lut_ft.py:59-79, and the save -> load -> dequantize round
trip against the hard quantizer that produced the bitstreams."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _say(msg):
    print(msg, flush=True)


def _signs(n, seed):
    return np.random.default_rng(seed).choice([-1.0, 1.0], size=n).astype(np.float32)


def _codebook(bcjr_mod, kind):
    if kind == "hyb16":
        lut = np.random.default_rng(2).standard_normal((1 << 9, 2)).astype(np.float32)
        return bcjr_mod.make_hyb_codebook_gpu(lut, 9, 16, "cuda")
    if kind == "3inst16":
        return bcjr_mod.make_3inst_codebook(16, "cuda")
    if kind == "1mad12":
        return bcjr_mod.make_1mad_codebook(12, "cuda")
    if kind == "table9v2":  # odd L, plain table
        return torch.tensor(np.random.default_rng(9).standard_normal((1 << 9, 2)).astype(np.float32), device="cuda")
    raise ValueError(kind)


def _payload(kind, cb, m, n, seed, Tx=16, Ty=16, k=2):
    L = int(cb.shape[0]).bit_length() - 1
    V = cb.shape[1]
    KV = k * V
    rng = np.random.default_rng(seed)
    nc, nr, N = n // Ty, m // Tx, Tx * Ty // V
    return {
        "bitstreams": rng.integers(0, 1 << KV, (nc, nr, N)).astype(np.uint8),
        "start_states": rng.integers(0, 1 << L, (nc, nr)).astype(np.int32),
        "sign_l": np.sign(rng.standard_normal(m)).astype(np.int8),
        "sign_r": np.sign(rng.standard_normal(n)).astype(np.int8),
        "W_scale": float(rng.uniform(0.005, 0.05)),
        "shape": (m, n),
        "meta": {"layer": 0, "kind": "attention", "proj": kind},
        "config": {"L": L, "k": k, "V": V, "Tx": Tx, "Ty": Ty},
    }


CASES = [("hyb16", 64, 256), ("3inst16", 128, 64), ("1mad12", 32, 512), ("table9v2", 48, 80)]


@pytest.mark.parametrize("kind,m,n", CASES)
def test_dequant_rotated_bit_exact(bcjr_mod, oracle, kind, m, n):
    """The rotated-basis matrix fl32(W_scale * c(walk)) from uint8, int32 and packed
    bitstreams equals the oracle's float64 product cast to float32, bit for bit."""
    from bcjr.serialize import dequant_target_gpu, pack_bitstreams
    _say(f"dequant rotated {kind} {m}x{n}")
    cb = _codebook(bcjr_mod, kind)
    p = _payload(kind, cb, m, n, seed=m + n)
    c = p["config"]
    ref = (oracle.dequant_unit(p["bitstreams"], p["start_states"], cb.cpu().numpy(), (m, n), c["L"],
                               c["k"] * c["V"], c["Tx"], c["Ty"]) * p["W_scale"]).astype(np.float32)
    got_u8 = dequant_target_gpu(p, rotated=True, codebook=cb)
    assert np.array_equal(got_u8.cpu().numpy(), ref)
    p32 = dict(p, bitstreams=p["bitstreams"].astype(np.int32))
    assert torch.equal(dequant_target_gpu(p32, rotated=True, codebook=cb), got_u8)
    pk = {kk: v for kk, v in p.items() if kk != "bitstreams"}
    pk["packed"] = pack_bitstreams(p["bitstreams"], c["k"] * c["V"])
    pk["n_steps"] = p["bitstreams"].shape[-1]
    assert torch.equal(dequant_target_gpu(pk, rotated=True, codebook=cb), got_u8)


@pytest.mark.parametrize("kind,m,n", [("hyb16", 64, 256), ("3inst16", 128, 128), ("hyb16", 512, 2048)])
def test_dequant_target_matches_oracle(bcjr_mod, oracle, kind, m, n):
    """dequant_target (float64 numpy, as the reference returns it) against the oracle;
    m*n an even power of two, so the inverse RHT's scale is exact and the match is
    bit-exact.  decode_fn (the reference's codebook callable) and a codebook tensor
    give the same result."""
    import bcjr
    _say(f"dequant_target {kind} {m}x{n}")
    cb = _codebook(bcjr_mod, kind)
    cb_np = cb.cpu().numpy()
    p = _payload(kind, cb, m, n, seed=3 * m + n)
    c = p["config"]
    ref = oracle.dequant_target(p["bitstreams"], p["start_states"], cb_np, p["sign_l"], p["sign_r"],
                                p["W_scale"], (m, n), c["L"], c["k"] * c["V"], c["Tx"], c["Ty"])
    got = bcjr.dequant_target(p, codebook=cb)
    assert got.dtype == np.float64 and got.shape == (m, n)
    assert np.array_equal(got, ref.astype(np.float64))
    got_fn = bcjr.dequant_target(p, lambda s: cb_np[s.astype(np.int64)])
    assert np.array_equal(got_fn, got)


def test_dequant_odd_power_shape(bcjr_mod, oracle):
    """m*n an odd power of two: the inverse RHT's 1/sqrt(mn) is inexact; within 2 ulp."""
    import bcjr
    _say("dequant_target 64x128")
    cb = _codebook(bcjr_mod, "3inst16")
    p = _payload("3inst16", cb, 64, 128, seed=5)
    ref = oracle.dequant_target(p["bitstreams"], p["start_states"], cb.cpu().numpy(), p["sign_l"], p["sign_r"],
                                p["W_scale"], (64, 128), 16, 2, 16, 16)
    got = bcjr.dequant_target(p, codebook=cb)
    assert np.abs(got - ref).max() <= 2 * np.spacing(np.abs(ref).max().astype(np.float32))


@pytest.mark.parametrize("kind,m,n,packed", [("3inst16", 128, 256, False), ("hyb16", 256, 128, True)])
def test_save_load_dequant_round_trip_equals_hard_quantizer(bcjr_mod, kind, m, n, packed, tmp_path):
    """Quantize with the Viterbi kernel, store the bitstreams in either format, load,
    dequantize: the result is the hard quantizer's W_q (quantize_forward_gpu), bit
    for bit (both multiply two float32 values and round once)."""
    import bcjr
    from bcjr.quant import tile_for_viterbi
    _say(f"round trip {kind} {m}x{n} packed={packed}")
    cb = _codebook(bcjr_mod, kind)
    V = cb.shape[1]
    sl = torch.tensor(_signs(m, 21), device="cuda")
    sr = torch.tensor(_signs(n, 22), device="cuda")
    W = torch.randn(m, n, device="cuda") * 0.03
    Wq = bcjr.quantize_forward_gpu(W, sl, sr, cb)
    Wt = bcjr.apply_rht_gpu(W, sl, sr)
    s = Wt.pow(2).mean().sqrt().clamp(min=1e-30)
    seqs, (nr, nc) = tile_for_viterbi(Wt / s, 16, 16)
    bits, start, _, _ = bcjr.viterbi_encode_v_batched_hip(seqs.contiguous(), cb, L=16, k=2, V=V)
    args = dict(bitstreams=bits.cpu().numpy().reshape(nc, nr, -1), start_states=start.cpu().numpy().reshape(nc, nr),
                sign_l=sl.cpu().numpy(), sign_r=sr.cpu().numpy(), W_scale=float(s), shape=(m, n),
                meta={"layer": 1, "kind": "mlp", "proj": "up_proj"}, config={"L": 16, "k": 2, "V": V, "Tx": 16, "Ty": 16})
    path = str(tmp_path / ("w.safetensors" if packed else "w.pt"))
    (bcjr.save_packed if packed else bcjr.save_quantized)(path, **args)
    d = bcjr.load_quantized(path)
    got = bcjr.dequant_target_gpu(d, codebook=cb)
    assert torch.equal(got, Wq)


def test_precompute_walk_states_bit_exact(bcjr_mod, oracle):
    import bcjr
    _say("walk states")
    rng = np.random.default_rng(4)
    for L, kV in [(16, 4), (16, 2), (9, 2), (11, 1)]:
        bits = rng.integers(0, 1 << kV, (3, 5, 128)).astype(np.uint8)
        start = rng.integers(0, 1 << L, (3, 5)).astype(np.int32)
        got = bcjr.precompute_walk_states(bits, start, L_bits=L, kV=kV)
        assert got.dtype == np.int64
        assert np.array_equal(got, oracle.walk_states(bits, start, L, kV))


def test_dequant_full_size_properties(bcjr_mod):
    """At a Llama-3.2-1B MLP shape (2048 x 8192, 65536 tiles): the three bitstream
    layouts agree, and dequantizing Viterbi output reproduces its reconstruction."""
    import bcjr
    from bcjr import ops
    from bcjr.quant import tile_for_viterbi, untile_from_viterbi
    from bcjr.serialize import pack_bitstreams
    _say("dequant 2048x8192")
    m, n = 2048, 8192
    cb = _codebook(bcjr_mod, "hyb16")
    W = torch.randn(m, n, device="cuda")
    seqs, info = tile_for_viterbi(W, 16, 16)
    bits, start, recon, _ = bcjr.viterbi_encode_v_batched_hip(seqs.contiguous(), cb, L=16, k=2, V=2)
    spec = ops.Spec(16, 2, 2, ops.CODE_HYB, 9)
    lut = cb._bcjr_lut
    scale = 0.0217
    a = ops.dequant(spec, start, lut, m, n, 16, 16, scale, bitstream=bits)
    b = ops.dequant(spec, start, lut, m, n, 16, 16, scale, bitstream=bits.to(torch.uint8))
    packed = torch.from_numpy(pack_bitstreams(bits.cpu().numpy(), 4)).cuda()
    c = ops.dequant(spec, start, lut, m, n, 16, 16, scale, packed=packed)
    assert torch.equal(a, b) and torch.equal(a, c)
    ref = (untile_from_viterbi(recon, info, (m, n), 16, 16).double() * scale).float()
    assert torch.equal(a, ref)


def test_dequant_empty_and_errors(bcjr_mod):
    from bcjr import ops
    from bcjr._lib import BcjrError
    _say("dequant empty / errors")
    spec = ops.Spec(16, 2, 1, ops.CODE_3INST)
    out = ops.dequant(spec, torch.zeros(0, dtype=torch.int32, device="cuda"), None, 0, 32, 16, 16, 1.0,
                      bitstream=torch.zeros(0, 256, dtype=torch.uint8, device="cuda"))
    assert out.shape == (0, 32)
    with pytest.raises(BcjrError, match="B=3"):
        ops.dequant(spec, torch.zeros(3, dtype=torch.int32, device="cuda"), None, 32, 32, 16, 16, 1.0,
                    bitstream=torch.zeros(3, 256, dtype=torch.uint8, device="cuda"))


@pytest.mark.parametrize("Tx,Ty,m,n", [(8, 2, 16, 6), (8, 12, 24, 36), (4, 8, 12, 40), (16, 16, 16, 16)])
def test_dequant_tile_shapes(bcjr_mod, oracle, Tx, Ty, m, n):
    """Tiles other than 16x16: Ty % 4 != 0 (scalar kernel), Ty not a power of two
    (vector kernel with divisions), and a single tile."""
    from bcjr.serialize import dequant_target_gpu
    _say(f"dequant tiles {Tx}x{Ty} of {m}x{n}")
    cb = _codebook(bcjr_mod, "table9v2")
    p = _payload("table9v2", cb, m, n, seed=Tx * Ty + m, Tx=Tx, Ty=Ty)
    ref = (oracle.dequant_unit(p["bitstreams"], p["start_states"], cb.cpu().numpy(), (m, n), 9, 4, Tx, Ty)
           * p["W_scale"]).astype(np.float32)
    assert np.array_equal(dequant_target_gpu(p, rotated=True, codebook=cb).cpu().numpy(), ref)
